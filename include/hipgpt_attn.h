#pragma once
// hipgpt_attn.h -- C ABI of the MI355X attention forward library
// (libhipgpt_attn.so).  Plain pointers and sizes; no C++ or torch types.
//
// Every entry point is asynchronous on the given stream (0 = null stream),
// allocates nothing unless stated, and returns HIPGPT_OK or a negative
// status (see hipgpt_attn_strerror).  Pointers are device pointers.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    HIPGPT_OK = 0,
    HIPGPT_ERR_INVALID = -1,      /* bad size, stride, pointer or flag        */
    HIPGPT_ERR_UNSUPPORTED = -2,  /* valid problem this build has no kernel for */
    HIPGPT_ERR_LAUNCH = -3,       /* the HIP launch itself failed             */
    HIPGPT_ERR_WORKSPACE = -4,    /* workspace missing or too small           */
    HIPGPT_ERR_SCRATCH = -5       /* beyond the no-allocation entry's scratch */
};

enum { HIPGPT_F32 = 0, HIPGPT_BF16 = 1 };

/* Output layouts of hipgpt_qkv_projection. */
enum { HIPGPT_QKV_ROWS = 0, HIPGPT_QKV_PLANAR = 1 };

/* Text for a status code. */
const char* hipgpt_attn_strerror(int status);

/* C-linkage twin of launch_multihead_attention (include/hip_kernels.h), for
 * FFI callers that cannot bind a C++ symbol.  Same contract, including the
 * abort on H <= 0 or E % H != 0.  Replaces src/hip_kernels.cpp:404-451. */
void hipgpt_launch_multihead_attention(const float* d_qkv, float* d_output,
                                       float* d_attn_probs, int B, int S,
                                       int E, int H);

/* C-linkage twins of HipGPT's unfused helpers (include/hip_kernels.h:44-46),
 * same contract as the C++ symbols declared in include/hip_kernels.h. */
void hipgpt_launch_scaled_dot_product(const float* Q, const float* K,
                                      float* scores, int B, int S, int D);
void hipgpt_launch_softmax(const float* scores, float* softmax_out, int B,
                           int S);
void hipgpt_launch_attention_weighted_sum(const float* softmax, const float* V,
                                          float* output, int B, int S, int D);

/* C-linkage twin of launch_multihead_attention_backward
 * (include/hip_kernels.h; replaces src/hip_kernels.cpp:1159-1272). */
void hipgpt_launch_multihead_attention_backward(const float* d_grad_attn_output,
                                                const float* d_qkv,
                                                const float* d_softmax,
                                                float* d_grad_qkv, int B, int S,
                                                int E, int H);

/* Backward with a caller-owned workspace (hipgpt_attn_bwd_workspace_bytes:
 * B*H*S floats), a stream, and a causal flag that skips tiles of the probs
 * wholly above the diagonal (a causal forward wrote zeros there).  Same
 * buffers as the drop-in; returns a status. */
size_t hipgpt_attn_bwd_workspace_bytes(int B, int S, int H);
int hipgpt_attn_bwd_qkv_planar(const float* grad_out, const float* qkv,
                               const float* probs, float* grad_qkv, int B,
                               int S, int E, int H, int causal,
                               void* workspace, size_t workspace_bytes,
                               hipStream_t stream);

/* No counterpart in HipGPT.  hipgpt_attn_bwd_qkv_planar without a workspace
 * argument, for callers that cannot allocate: code under HIP graph capture,
 * tight serving/training loops, harnesses that forbid hipMalloc.  It calls no
 * allocator; its B*H*S row-dot workspace is a fixed 4 MiB array per GPU
 * inside the library, so B*H*S must be at most 1048576 (else
 * HIPGPT_ERR_SCRATCH, nothing launched).  Calls that overlap on one GPU (two
 * streams, or host threads) share that array and race; serialise them.
 * Results are identical to hipgpt_attn_bwd_qkv_planar's. */
int hipgpt_attn_bwd_qkv_planar_noalloc(const float* grad_out, const float* qkv,
                                       const float* probs, float* grad_qkv,
                                       int B, int S, int E, int H, int causal,
                                       hipStream_t stream);

/* Training pair without the [B][H][S][S] probs buffer (FlashAttention-2's
 * forward/backward split).  No counterpart in HipGPT, whose backward reads the
 * stored probs (src/hip_kernels.cpp:1159-1272); this pair computes the same
 * gradients from O and a per-row log-sum-exp instead.
 *   forward:  planar buffers as hipgpt_attn_qkv_planar, plus
 *             lse [B][H][S] = ln sum_j exp(q_i . k_j / sqrt(D)) over the keys
 *             query i sees (all, or j <= i when causal).
 *   backward: grad_out, qkv, the forward's out and lse -> every element of
 *             the planar grad_qkv [dQ|dK|dV]; P is recomputed per tile.
 *             At D = 32 and 64 workspace / workspace_bytes are ignored (may
 *             be NULL / 0); other head dims need the B*H*S floats of
 *             hipgpt_attn_bwd_workspace_bytes (else HIPGPT_ERR_WORKSPACE).
 * fp32, D = E/H a multiple of 4 up to 256, 16-byte aligned buffers; other
 * shapes return HIPGPT_ERR_UNSUPPORTED. */
int hipgpt_attn_fwd_lse_qkv_planar(const float* d_qkv, float* d_output,
                                   float* lse, int B, int S, int E, int H,
                                   int causal, hipStream_t stream);
int hipgpt_attn_bwd_lse_qkv_planar(const float* grad_out, const float* qkv,
                                   const float* out, const float* lse,
                                   float* grad_qkv, int B, int S, int E, int H,
                                   int causal, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream);

/* HipGPT's planar [3][B*S][E] layout with the options the legacy symbol
 * lacks: causal masking (keys j <= i; probs written 0 above the diagonal so
 * HipGPT's backward, src/hip_kernels.cpp:1162-1243, stays exact) and a
 * stream.  Returns a status instead of aborting. */
int hipgpt_attn_qkv_planar(const float* d_qkv, float* d_output,
                           float* d_attn_probs, int B, int S, int E, int H,
                           int causal, hipStream_t stream);

/* General strided attention forward.
 *   q, k, v: element (b, s, h, d) at X[b*x_bs + s*x_ts + h*x_hs + d], in
 *            `dtype` (HIPGPT_F32 or HIPGPT_BF16); d is contiguous.
 *   o:       fp32, same indexing with o_* strides.
 *   probs:   optional dense fp32 [B][H][Sq][Sk] normalised probabilities.
 *   scale:   softmax scale; <= 0 selects 1/sqrt(D).
 *   causal:  query i sees keys j <= i + (Sk - Sq); requires Sk >= Sq.
 * bf16 inputs are computed with bf16 MFMA and fp32 accumulation, D in
 * {32, 64, 128}, 16-byte aligned rows (strides multiple of 8). */
int hipgpt_attn_fwd(const void* q, const void* k, const void* v, float* o,
                    float* probs, int B, int H, int Sq, int Sk, int D,
                    int64_t q_bs, int64_t q_ts, int64_t q_hs,
                    int64_t k_bs, int64_t k_ts, int64_t k_hs,
                    int64_t v_bs, int64_t v_ts, int64_t v_hs,
                    int64_t o_bs, int64_t o_ts, int64_t o_hs,
                    float scale, int causal, int dtype, hipStream_t stream);

/* Single-query decode step: q [B][1][..] attends to kv_len keys (all
 * visible).  Split-KV: num_splits partial workgroups per (b, h) write
 * (max, sum, O) to `workspace`, a reduce kernel merges them.
 * num_splits <= 0 picks hipgpt_attn_decode_default_splits().  fp32, D in
 * {32, 64, 128, 256}, 16-byte aligned rows.  The workspace is caller-owned
 * device memory of hipgpt_attn_decode_workspace_bytes() bytes (may be NULL
 * when the split count is 1). */
int hipgpt_attn_decode_default_splits(int B, int H, int kv_len);
size_t hipgpt_attn_decode_workspace_bytes(int B, int H, int D, int num_splits);
int hipgpt_attn_decode(const float* q, const float* k, const float* v,
                       float* o, int B, int H, int kv_len, int D,
                       int64_t q_bs, int64_t q_hs,
                       int64_t k_bs, int64_t k_ts, int64_t k_hs,
                       int64_t v_bs, int64_t v_ts, int64_t v_hs,
                       int64_t o_bs, int64_t o_hs,
                       float scale, int num_splits, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);

/* One KV-cached decode step for a batch of sequences of different lengths
 * (the step HipGPT's generation loop, src/gpt_model.cpp:261-273, would take
 * instead of recomputing the whole window per token).
 *   k_cache, v_cache: [B][max_len][H][D] fp32, element (b, t, h, d) at
 *     X[b*c_bs + t*c_ts + h*c_hs + d]; rows [0, lens[b]) hold the cached
 *     keys / values of sequence b.
 *   lens: device int32 [B], read on the device (no host synchronisation).
 *   q, k_new, v_new, o: the step's rows [B][H][D] with (bs, hs) strides.
 * The step writes k_new / v_new into row lens[b] of the caches, computes
 * o = softmax(q K^T * scale) V over the lens[b] + 1 rows, and, when advance
 * is non-zero, increments lens[b].  A sequence with lens[b] < 0 or
 * lens[b] >= max_len is left unchanged and gets a NaN output.  Split-KV as
 * hipgpt_attn_decode (num_splits <= 0 picks the default for max_len; the
 * workspace is hipgpt_attn_decode_workspace_bytes(B, H, D, splits)).  fp32,
 * D in {32, 64, 128, 256}, 16-byte aligned rows.  Rows past lens[b] + 1 are
 * never read. */
int hipgpt_attn_decode_kvcache(const float* q, const float* k_new,
                               const float* v_new, float* k_cache,
                               float* v_cache, int* lens, float* o, int B,
                               int H, int D, int max_len,
                               int64_t q_bs, int64_t q_hs,
                               int64_t kn_bs, int64_t kn_hs,
                               int64_t vn_bs, int64_t vn_hs,
                               int64_t c_bs, int64_t c_ts, int64_t c_hs,
                               int64_t o_bs, int64_t o_hs, float scale,
                               int num_splits, int advance, void* workspace,
                               size_t workspace_bytes, hipStream_t stream);

/* Diagnostics, no counterpart in HipGPT.  Two kernels synchronise their waves
 * through LDS flags instead of barriers (the resident-K/V forward at D = 64,
 * S <= 256, and the one-workgroup-per-(b, h) backward at D = 32, S <= 256).
 * Their waits are bounded so a fault in the schedule cannot hang the GPU; a
 * wait that runs out is counted on the device.  *count receives the number
 * of expired waits on the current device since the last clear (zero in a
 * correct run; non-zero means some outputs may be wrong).  clear != 0 resets
 * the count in the same device-side atomic that reads it.  Blocking: a
 * one-thread kernel and a copy on the null stream.  The count is exact only
 * when no library kernel is in flight on another stream (the null stream does
 * not wait for non-blocking streams): synchronise the device first. */
int hipgpt_attn_wait_expired(unsigned int* count, int clear);

/* ---- projections either side of the attention (fp32 MFMA GEMM) ---- */

/* C-linkage twins of launch_matmul / launch_matmul_add_bias
 * (include/hip_kernels.h; replace src/hip_kernels.cpp:70-154). */
void hipgpt_launch_matmul(const float* A, const float* B, float* C, int M,
                          int N, int K);
void hipgpt_launch_matmul_add_bias(const float* A, const float* B,
                                   const float* bias, float* C, int M, int N,
                                   int K);

/* General GEMM + bias: C[m][n] = sum_k A[m][k] W[k][n] (+ bias[n]).
 *   A [M][K] row stride lda; W [K][N] row stride ldw; bias [N] or NULL.
 *   Output column n is stored at C + (n / seg_w) * seg_stride + m * ldc
 *   + n % seg_w (elements of out_dtype): seg_w = N gives a row-major [M][N]
 *   buffer; seg_w = N/3, seg_stride = M*N/3 splits a QKV projection into
 *   planar [3][M][N/3].  out_dtype HIPGPT_F32 or HIPGPT_BF16 (RNE).
 *   Requires M, N >= 1, K >= 0, lda >= K, ldw >= N, 1 <= seg_w <= N,
 *   ldc >= seg_w, seg_stride >= 0. */
int hipgpt_gemm_bias(const float* A, const float* W, const float* bias,
                     void* C, int M, int N, int K, int64_t lda, int64_t ldw,
                     int64_t ldc, int seg_w, int64_t seg_stride,
                     int out_dtype, hipStream_t stream);

/* HipGPT's QKV projection (src/transformer_layer.cpp:217): x [T][E] times
 * w_qkv [E][3E] plus b_qkv [3E].  layout HIPGPT_QKV_ROWS writes the
 * reference's [T][3E] buffer; HIPGPT_QKV_PLANAR writes [3][T][E], so that
 * plane p row t is projection p of token t in the layout the attention
 * launchers read.  out_dtype HIPGPT_F32 or HIPGPT_BF16. */
int hipgpt_qkv_projection(const float* x, const float* w_qkv,
                          const float* b_qkv, void* out, int T, int E,
                          int layout, int out_dtype, hipStream_t stream);

#ifdef __cplusplus
}
#endif
