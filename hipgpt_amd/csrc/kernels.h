// kernels.h -- internal launch functions shared by the C ABI (api.cpp) and the
// kernel translation units.  Not installed; the public surface is
// include/hip_kernels.h and include/hipgpt_attn.h.
#pragma once

#include "common.h"

namespace hipgpt {

// Padded head dim served by the fp32 MFMA kernel (32, 64, 128), 0 if none.
int fa_f32_padded_dim(int D);
// fp32 MFMA flash attention.  vec: D equals the padded dim and every stride
// and base pointer allows 16-byte accesses.
hipError_t launch_fa_f32(const AttnArgs& a, bool causal, bool vec, hipStream_t stream);

// bf16-input / fp32-accumulate MFMA flash attention (D in {32, 64, 128},
// 16-byte aligned rows).  Writes fp32 O (and fp32 probs when requested).
bool fa_bf16_supported(int D);
hipError_t launch_fa_bf16(const AttnArgs& a, bool causal, hipStream_t stream);

// fp32 MFMA attention for 128 < D <= 256 with D % 4 == 0 (head dim split over
// four waves per query sub-block); needs 16-byte aligned rows.
bool fa_wide_supported(int D);
hipError_t launch_fa_wide(const AttnArgs& a, bool causal, hipStream_t stream);

// Any head dim, fp32: one wave per query row (the path for other D > 128).
hipError_t launch_attn_generic_f32(const AttnArgs& a, bool causal, hipStream_t stream);

// Expired bounded waits (note_wait_expired) of the kernels in fa_f32.hip (the
// resident-K/V forward) and bwd.hip (the per-(b, h) backward) on the current
// device; cleared after the read when `clear` is set.
hipError_t fa_f32_wait_expired(unsigned int* count, bool clear);
hipError_t bwd_wait_expired(unsigned int* count, bool clear);

// KV-cache decode step: the cache is a.k / a.v (with a.k_* / a.v_* strides,
// a.Sk = max_len); the new row of sequence b is appended at lens[b].
struct KvcArgs {
    const float* k_new;
    const float* v_new;
    int64_t kn_bs, kn_hs, vn_bs, vn_hs;
    float* kc;  // writable views of the caches (same memory as a.k / a.v)
    float* vc;
    int* lens;  // device [B]
    int max_len;
    int advance;  // increment lens[b] after the step
};

// Split-KV single-query decode.  q: [B][1][H*D]-style strides in a; partial
// results go to ws (nsplit * B * H * (D + 2) floats) when nsplit > 1.
// kc != null selects the KV-cache step.
bool decode_supported(int D, int dtype);
int decode_default_splits(int B, int H, int kv_len);
hipError_t launch_decode(const AttnArgs& a, int dtype, int nsplit, float* ws, hipStream_t stream,
                         const KvcArgs* kc = nullptr);

// Attention backward on the forward's probs (HipGPT src/hip_kernels.cpp:1159-1272).
// All [B][S][H][D] tensors share one (batch, token, head) stride set; dvec is
// a B*H*S float workspace (row dots dO_i . (P V)_i).
struct BwdArgs {
    const float *q, *k, *v, *go, *probs;
    float *dq, *dk, *dv, *dvec;
    // Recompute mode (probs == nullptr): the forward's output O and row
    // log-sum-exp lse [B*H][S] (natural log); P is rebuilt per tile as
    // exp(scale q.k - lse) and the row dots dO . O are formed from dO and O
    // (dvec is unused).
    const float *o, *lse;
    int64_t bs, ts, hs;
    int B, H, S, D;
    int causal;
    float scale;
    // Set by the launcher: workgroups the device holds at once for the chosen
    // kernel, capped at the grid (0 = unknown); the per-(b, h) kernel's
    // staggered start is timed for, and applied to, that first set.
    int resident;
};
hipError_t launch_attn_bwd(const BwdArgs& a, hipStream_t s);
// The per-wave LDS-tiled MFMA kernels apply (D = 32 or 64, 16-byte aligned rows).
bool bwd_tiled_ok(const BwdArgs& a);
// Recompute mode (a.o, a.lse, no probs) has a kernel: the tiled ones, or the
// head-dim-split ones (D % 4 == 0 up to 256, 16-byte aligned rows).
bool bwd_recompute_ok(const BwdArgs& a);
// False when launch_attn_bwd takes a path that needs no dvec workspace (the
// one-workgroup-per-(b, h) kernels, or recompute mode at D = 32 / 64).
bool bwd_uses_workspace(const BwdArgs& a);

// Unfused single-head helpers (HipGPT src/hip_kernels.cpp:454-532).
hipError_t launch_sdp(const float* Q, const float* K, float* scores, int B, int S, int D, hipStream_t s);
hipError_t launch_softmax_rows(const float* in, float* out, int B, int S, hipStream_t s);
hipError_t launch_wsum(const float* P, const float* V, float* O, int B, int S, int D, hipStream_t s);

// fp32 GEMM + bias (HipGPT src/hip_kernels.cpp:70-154):
//   C[m][n] = sum_k A[m][k] W[k][n] (+ bias[n]), output column n stored at
//   C + (n / seg_w) * seg_stride + m * ldc + n % seg_w, fp32 or bf16.
struct GemmArgs {
    const float* A;
    const float* W;
    const float* bias;  // may be null
    void* C;
    int M, N, K;
    int64_t lda, ldw, ldc;
    int seg_w;
    int64_t seg_stride;
    int out_bf16;
};
// True when the 16-byte vector path applies (alignment, multiples of 4).
bool gemm_vec_ok(const GemmArgs& g);
hipError_t launch_gemm(const GemmArgs& g, hipStream_t s);

}  // namespace hipgpt
