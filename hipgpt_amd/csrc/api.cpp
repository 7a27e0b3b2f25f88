// api.cpp -- host side of libhipgpt_attn.so: validation, kernel selection,
// the drop-in launch_multihead_attention and the C ABI of hipgpt_attn.h.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "../../include/hip_kernels.h"
#include "../../include/hipgpt_attn.h"
#include "kernels.h"

using hipgpt::AttnArgs;

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

float default_scale(int D, float scale) { return scale > 0.f ? scale : 1.0f / std::sqrt((float)D); }

int from_hip(hipError_t e) { return e == hipSuccess ? HIPGPT_OK : HIPGPT_ERR_LAUNCH; }

// The MFMA kernels address a (batch, head) slice of K and V with 32-bit byte
// offsets (buffer loads), including up to a few tiles past the last row.
bool kv_slice_fits_32bit(const AttnArgs& a, int elem_bytes) {
    const int64_t ts = a.k_ts > a.v_ts ? a.k_ts : a.v_ts;
    return ((int64_t)(a.Sk + 256) * ts + a.D) * elem_bytes < ((int64_t)1 << 31);
}

// Shared validation and dispatch for every forward entry point.
int attn_dispatch(const AttnArgs& in, int causal, int dtype, hipStream_t stream) {
    if (!in.q || !in.k || !in.v || !in.o) return HIPGPT_ERR_INVALID;
    if (in.B <= 0 || in.H <= 0 || in.Sq <= 0 || in.Sk <= 0 || in.D <= 0) return HIPGPT_ERR_INVALID;
    if (causal && in.Sk < in.Sq) return HIPGPT_ERR_INVALID;
    if (dtype != HIPGPT_F32 && dtype != HIPGPT_BF16) return HIPGPT_ERR_INVALID;
    if ((int64_t)in.B * in.H > 0x7fffffff) return HIPGPT_ERR_INVALID;
    AttnArgs a = in;
    a.causal_off = causal ? in.Sk - in.Sq : 0;

    if (dtype == HIPGPT_BF16) {
        if (!hipgpt::fa_bf16_supported(a.D)) return HIPGPT_ERR_UNSUPPORTED;
        const bool ok = aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.o) &&
                        a.q_bs % 8 == 0 && a.q_ts % 8 == 0 && a.q_hs % 8 == 0 && a.k_bs % 8 == 0 &&
                        a.k_ts % 8 == 0 && a.k_hs % 8 == 0 && a.v_bs % 8 == 0 && a.v_ts % 8 == 0 &&
                        a.v_hs % 8 == 0 && a.o_bs % 4 == 0 && a.o_ts % 4 == 0 && a.o_hs % 4 == 0;
        if (!ok || !kv_slice_fits_32bit(a, 2)) return HIPGPT_ERR_UNSUPPORTED;
        return from_hip(hipgpt::launch_fa_bf16(a, causal != 0, stream));
    }

    // 16-byte rows: aligned bases and strides, K / V slices within 2^31 bytes
    const bool rows16 = aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.o) &&
                        a.q_bs % 4 == 0 && a.q_ts % 4 == 0 && a.q_hs % 4 == 0 && a.k_bs % 4 == 0 &&
                        a.k_ts % 4 == 0 && a.k_hs % 4 == 0 && a.v_bs % 4 == 0 && a.v_ts % 4 == 0 &&
                        a.v_hs % 4 == 0 && a.o_bs % 4 == 0 && a.o_ts % 4 == 0 && a.o_hs % 4 == 0 &&
                        kv_slice_fits_32bit(a, 4);
    const int dp = hipgpt::fa_f32_padded_dim(a.D);
    if (dp == 0) {
        if (hipgpt::fa_wide_supported(a.D) && rows16) return from_hip(hipgpt::launch_fa_wide(a, causal != 0, stream));
        return from_hip(hipgpt::launch_attn_generic_f32(a, causal != 0, stream));
    }
    const bool vec = a.D == dp && rows16 && (!a.probs || aligned16(a.probs));
    return from_hip(hipgpt::launch_fa_f32(a, causal != 0, vec, stream));
}

// The planar [3][B*S][E] buffer of src/hip_kernels.cpp:415-417 as strides.
AttnArgs planar_args(const float* qkv, float* out, float* probs, int B, int S, int E, int H) {
    const int64_t plane = (int64_t)B * S * E;
    AttnArgs a{};
    a.q = qkv;
    a.k = qkv + plane;
    a.v = qkv + 2 * plane;
    a.o = out;
    a.probs = probs;
    a.q_bs = a.k_bs = a.v_bs = a.o_bs = (int64_t)S * E;
    a.q_ts = a.k_ts = a.v_ts = a.o_ts = E;
    a.q_hs = a.k_hs = a.v_hs = a.o_hs = E / H;
    a.B = B;
    a.H = H;
    a.Sq = S;
    a.Sk = S;
    a.D = E / H;
    a.qscale = default_scale(a.D, 0.f) * hipgpt::kLog2e;
    return a;
}

}  // namespace

// ------------------------------------------------------------ drop-in symbol

void launch_multihead_attention(const float* d_qkv, float* d_output, float* d_attn_probs, int B, int S,
                                int E, int H) {
    if (H <= 0 || (E % H) != 0) {  // src/hip_kernels.cpp:410-413
        fprintf(stderr, "Bad MHA config: E=%d H=%d\n", E, H);
        abort();
    }
    if (B <= 0 || S <= 0 || E <= 0) return;  // nothing to launch (the reference's grid would be empty)
    const int rc = attn_dispatch(planar_args(d_qkv, d_output, d_attn_probs, B, S, E, H), 0, HIPGPT_F32, 0);
    if (rc != HIPGPT_OK)
        fprintf(stderr, "launch_multihead_attention: %s (B=%d S=%d E=%d H=%d)\n", hipgpt_attn_strerror(rc), B,
                S, E, H);
}

// Unfused helpers (src/hip_kernels.cpp:454-532): the reference launches them
// unchecked on the null stream; so do these (a failed launch is reported on
// stderr, as for the attention launcher).
static void report(hipError_t e, const char* what) {
    if (e != hipSuccess) fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
}

void launch_scaled_dot_product(const float* Q, const float* K, float* scores, int B, int S, int D) {
    if (B <= 0 || S <= 0 || D <= 0 || B > 65535) return;
    report(hipgpt::launch_sdp(Q, K, scores, B, S, D, 0), "launch_scaled_dot_product");
}

void launch_softmax(const float* scores, float* softmax_out, int B, int S) {
    if (B <= 0 || S <= 0) return;
    report(hipgpt::launch_softmax_rows(scores, softmax_out, B, S, 0), "launch_softmax");
}

void launch_attention_weighted_sum(const float* softmax, const float* V, float* output, int B, int S, int D) {
    if (B <= 0 || S <= 0 || D <= 0 || B > 65535) return;
    report(hipgpt::launch_wsum(softmax, V, output, B, S, D, 0), "launch_attention_weighted_sum");
}

// Attention backward (src/hip_kernels.cpp:1245-1272).  The planar buffers of
// the forward; the B*H*S row-dot workspace comes from the caller or, for the
// drop-in symbol (whose signature has no workspace), from a buffer cached per
// device and grown on demand -- only for shapes whose kernels use it (not,
// e.g., D = 32 with S <= 256, whose per-(b, h) kernel forms the row dots in
// LDS).
namespace {

hipgpt::BwdArgs planar_bwd_args(const float* go, const float* qkv, const float* probs, float* gqkv, int B, int S,
                                int E, int H, int causal) {
    const int64_t plane = (int64_t)B * S * E;
    hipgpt::BwdArgs a{};
    a.q = qkv;
    a.k = qkv + plane;
    a.v = qkv + 2 * plane;
    a.go = go;
    a.probs = probs;
    a.dq = gqkv;
    a.dk = gqkv + plane;
    a.dv = gqkv + 2 * plane;
    a.bs = (int64_t)S * E;
    a.ts = E;
    a.hs = E / H;
    a.B = B;
    a.H = H;
    a.S = S;
    a.D = E / H;
    a.causal = causal;
    a.scale = 1.0f / std::sqrt((float)a.D);
    return a;
}

// Guards the cached workspace from the lookup until the kernels that use it
// are enqueued, so a concurrent call that grows (frees) the buffer cannot
// free it between another thread's lookup and launch.
std::mutex& bwd_workspace_mutex() {
    static std::mutex mu;
    return mu;
}

// Caller holds bwd_workspace_mutex().  Grows the current device's buffer when
// too small (hipFree of the old one waits for the device to finish with it).
float* cached_bwd_workspace(size_t bytes) {
    static void* buf[64] = {};
    static size_t cap[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    if (cap[dev] < bytes) {
        if (buf[dev] && hipFree(buf[dev]) != hipSuccess) return nullptr;
        buf[dev] = nullptr;
        cap[dev] = 0;
        if (hipMalloc(&buf[dev], bytes) != hipSuccess) return nullptr;
        cap[dev] = bytes;
    }
    return static_cast<float*>(buf[dev]);
}

}  // namespace

void launch_multihead_attention_backward(const float* d_grad_attn_output, const float* d_qkv, const float* d_softmax,
                                         float* d_grad_qkv, int B, int S, int E, int H) {
    if (H <= 0 || (E % H) != 0) {  // the reference divides by H unchecked; abort as the forward does
        fprintf(stderr, "Bad MHA config: E=%d H=%d\n", E, H);
        abort();
    }
    if (B <= 0 || S <= 0 || E <= 0) return;
    hipgpt::BwdArgs a = planar_bwd_args(d_grad_attn_output, d_qkv, d_softmax, d_grad_qkv, B, S, E, H, 0);
    if (!hipgpt::bwd_uses_workspace(a)) {  // HipGPT's default shape (D = 32, S <= 256) needs none
        report(hipgpt::launch_attn_bwd(a, 0), "launch_multihead_attention_backward");
        return;
    }
    // Not capturable (it may allocate); hipgpt_attn_bwd_qkv_planar (caller
    // workspace) and hipgpt_attn_bwd_qkv_planar_noalloc are.
    std::lock_guard<std::mutex> lock(bwd_workspace_mutex());
    a.dvec = cached_bwd_workspace((size_t)B * H * S * sizeof(float));
    if (!a.dvec) {
        fprintf(stderr, "launch_multihead_attention_backward: workspace allocation failed\n");
        return;
    }
    report(hipgpt::launch_attn_bwd(a, 0), "launch_multihead_attention_backward");
}

// ------------------------------------------------- no-allocation backward
// Fixed per-device scratch of hipgpt_attn_bwd_qkv_planar_noalloc: the B*H*S
// row-dot workspace of the backward kernels (every element a call reads is
// written earlier in the same call, so nothing needs clearing).  Each GPU the
// library runs on holds its own copy until the process ends.  In host code
// `scratch` names a host-side stand-in, never the device memory: its device
// address comes from hipGetSymbolAddress, once per device (scratch_ptr).
constexpr size_t kScratchFloats = (size_t)1 << 20;  // 4 MiB
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {

// Device address of `scratch` on the current device, looked up on the first
// call on that device (with it current) and kept per device.
float* scratch_ptr() {
    static std::mutex mu;
    static float* ptr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        ptr[dev] = static_cast<float*>(p);
    }
    return ptr[dev];
}

}  // namespace

// GEMMs either side of the attention (src/hip_kernels.cpp:102-154): the
// reference's naming, A [M][N] x B [N][K] -> C [M][K].
namespace {

hipgpt::GemmArgs ref_gemm_args(const float* A, const float* B, const float* bias, float* C, int M, int N, int K) {
    hipgpt::GemmArgs g{};
    g.A = A;
    g.W = B;
    g.bias = bias;
    g.C = C;
    g.M = M;
    g.N = K;
    g.K = N > 0 ? N : 0;
    g.lda = N > 0 ? N : 0;
    g.ldw = K;
    g.ldc = K;
    g.seg_w = K;
    g.seg_stride = 0;
    g.out_bf16 = 0;
    return g;
}

}  // namespace

void launch_matmul(const float* A, const float* B, float* C, int M, int N, int K) {
    if (M <= 0 || K <= 0) return;  // the reference's grid would be empty
    report(hipgpt::launch_gemm(ref_gemm_args(A, B, nullptr, C, M, N, K), 0), "launch_matmul");
}

void launch_matmul_add_bias(const float* A, const float* B, const float* bias, float* C, int M, int N, int K) {
    if (M <= 0 || K <= 0) return;
    report(hipgpt::launch_gemm(ref_gemm_args(A, B, bias, C, M, N, K), 0), "launch_matmul_add_bias");
}

// ------------------------------------------------------------------- C ABI

extern "C" {

const char* hipgpt_attn_strerror(int status) {
    switch (status) {
        case HIPGPT_OK: return "ok";
        case HIPGPT_ERR_INVALID: return "invalid argument";
        case HIPGPT_ERR_UNSUPPORTED: return "unsupported problem (head dim, dtype or alignment)";
        case HIPGPT_ERR_LAUNCH: return "kernel launch failed";
        case HIPGPT_ERR_WORKSPACE: return "workspace missing or too small";
        case HIPGPT_ERR_SCRATCH: return "problem exceeds the fixed scratch of the no-allocation entry point";
        default: return "unknown status";
    }
}

void hipgpt_launch_multihead_attention(const float* d_qkv, float* d_output, float* d_attn_probs, int B,
                                       int S, int E, int H) {
    launch_multihead_attention(d_qkv, d_output, d_attn_probs, B, S, E, H);
}

void hipgpt_launch_scaled_dot_product(const float* Q, const float* K, float* scores, int B, int S, int D) {
    launch_scaled_dot_product(Q, K, scores, B, S, D);
}

void hipgpt_launch_softmax(const float* scores, float* softmax_out, int B, int S) {
    launch_softmax(scores, softmax_out, B, S);
}

void hipgpt_launch_attention_weighted_sum(const float* softmax, const float* V, float* output, int B, int S, int D) {
    launch_attention_weighted_sum(softmax, V, output, B, S, D);
}

void hipgpt_launch_multihead_attention_backward(const float* d_grad_attn_output, const float* d_qkv,
                                                const float* d_softmax, float* d_grad_qkv, int B, int S, int E,
                                                int H) {
    launch_multihead_attention_backward(d_grad_attn_output, d_qkv, d_softmax, d_grad_qkv, B, S, E, H);
}

size_t hipgpt_attn_bwd_workspace_bytes(int B, int S, int H) {
    if (B <= 0 || S <= 0 || H <= 0) return 0;
    return (size_t)B * H * S * sizeof(float);
}

int hipgpt_attn_bwd_qkv_planar(const float* grad_out, const float* qkv, const float* probs, float* grad_qkv, int B,
                               int S, int E, int H, int causal, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
    if (!grad_out || !qkv || !probs || !grad_qkv || B <= 0 || S <= 0 || E <= 0 || H <= 0 || E % H != 0)
        return HIPGPT_ERR_INVALID;
    if ((int64_t)B * H > 0x7fffffff) return HIPGPT_ERR_INVALID;
    if (!workspace || workspace_bytes < hipgpt_attn_bwd_workspace_bytes(B, S, H)) return HIPGPT_ERR_WORKSPACE;
    hipgpt::BwdArgs a = planar_bwd_args(grad_out, qkv, probs, grad_qkv, B, S, E, H, causal ? 1 : 0);
    a.dvec = static_cast<float*>(workspace);
    return from_hip(hipgpt::launch_attn_bwd(a, stream));
}

int hipgpt_attn_bwd_qkv_planar_noalloc(const float* grad_out, const float* qkv, const float* probs,
                                       float* grad_qkv, int B, int S, int E, int H, int causal,
                                       hipStream_t stream) {
    // The scratch limit is checked before the pointers, so a problem beyond
    // it is rejected whatever buffers come with it (nothing is launched).
    if (B <= 0 || S <= 0 || E <= 0 || H <= 0 || E % H != 0) return HIPGPT_ERR_INVALID;
    if ((int64_t)B * H > 0x7fffffff) return HIPGPT_ERR_INVALID;
    if ((uint64_t)B * (uint64_t)H * (uint64_t)S > kScratchFloats) return HIPGPT_ERR_SCRATCH;
    if (!grad_out || !qkv || !probs || !grad_qkv) return HIPGPT_ERR_INVALID;
    hipgpt::BwdArgs a = planar_bwd_args(grad_out, qkv, probs, grad_qkv, B, S, E, H, causal ? 1 : 0);
    if (hipgpt::bwd_uses_workspace(a)) {
        a.dvec = scratch_ptr();
        if (!a.dvec) return HIPGPT_ERR_LAUNCH;
    }
    return from_hip(hipgpt::launch_attn_bwd(a, stream));
}

int hipgpt_attn_fwd_lse_qkv_planar(const float* d_qkv, float* d_output, float* lse, int B, int S, int E, int H,
                                   int causal, hipStream_t stream) {
    if (!d_qkv || !d_output || !lse || B <= 0 || S <= 0 || E <= 0 || H <= 0 || E % H != 0) return HIPGPT_ERR_INVALID;
    const int D = E / H;
    if (D % 4 != 0 || D > 256 || !aligned16(d_qkv) || !aligned16(d_output)) return HIPGPT_ERR_UNSUPPORTED;
    AttnArgs a = planar_args(d_qkv, d_output, nullptr, B, S, E, H);
    a.lse = lse;
    return attn_dispatch(a, causal, HIPGPT_F32, stream);
}

int hipgpt_attn_bwd_lse_qkv_planar(const float* grad_out, const float* qkv, const float* out, const float* lse,
                                   float* grad_qkv, int B, int S, int E, int H, int causal, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
    if (!grad_out || !qkv || !out || !lse || !grad_qkv || B <= 0 || S <= 0 || E <= 0 || H <= 0 || E % H != 0)
        return HIPGPT_ERR_INVALID;
    if ((int64_t)B * H > 0x7fffffff) return HIPGPT_ERR_INVALID;
    hipgpt::BwdArgs a = planar_bwd_args(grad_out, qkv, nullptr, grad_qkv, B, S, E, H, causal ? 1 : 0);
    a.o = out;
    a.lse = lse;
    if (!hipgpt::bwd_recompute_ok(a)) return HIPGPT_ERR_UNSUPPORTED;
    // D = 32 / 64 form the row dots dO . O inside each kernel; the other head
    // dims pass them from the first kernel to the second through the workspace
    if (hipgpt::bwd_uses_workspace(a)) {
        if (!workspace || workspace_bytes < hipgpt_attn_bwd_workspace_bytes(B, S, H)) return HIPGPT_ERR_WORKSPACE;
        a.dvec = static_cast<float*>(workspace);
    }
    return from_hip(hipgpt::launch_attn_bwd(a, stream));
}

int hipgpt_attn_qkv_planar(const float* d_qkv, float* d_output, float* d_attn_probs, int B, int S, int E,
                           int H, int causal, hipStream_t stream) {
    if (!d_qkv || !d_output || B <= 0 || S <= 0 || E <= 0 || H <= 0 || E % H != 0) return HIPGPT_ERR_INVALID;
    return attn_dispatch(planar_args(d_qkv, d_output, d_attn_probs, B, S, E, H), causal, HIPGPT_F32, stream);
}

int hipgpt_attn_fwd(const void* q, const void* k, const void* v, float* o, float* probs, int B, int H, int Sq,
                    int Sk, int D, int64_t q_bs, int64_t q_ts, int64_t q_hs, int64_t k_bs, int64_t k_ts,
                    int64_t k_hs, int64_t v_bs, int64_t v_ts, int64_t v_hs, int64_t o_bs, int64_t o_ts,
                    int64_t o_hs, float scale, int causal, int dtype, hipStream_t stream) {
    if (D <= 0 || !std::isfinite(scale)) return HIPGPT_ERR_INVALID;
    AttnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.probs = probs;
    a.q_bs = q_bs;
    a.q_ts = q_ts;
    a.q_hs = q_hs;
    a.k_bs = k_bs;
    a.k_ts = k_ts;
    a.k_hs = k_hs;
    a.v_bs = v_bs;
    a.v_ts = v_ts;
    a.v_hs = v_hs;
    a.o_bs = o_bs;
    a.o_ts = o_ts;
    a.o_hs = o_hs;
    a.B = B;
    a.H = H;
    a.Sq = Sq;
    a.Sk = Sk;
    a.D = D;
    a.qscale = default_scale(D, scale) * hipgpt::kLog2e;
    return attn_dispatch(a, causal, dtype, stream);
}

int hipgpt_attn_decode_default_splits(int B, int H, int kv_len) {
    if (B <= 0 || H <= 0 || kv_len <= 0) return 1;
    return hipgpt::decode_default_splits(B, H, kv_len);
}

size_t hipgpt_attn_decode_workspace_bytes(int B, int H, int D, int num_splits) {
    if (B <= 0 || H <= 0 || D <= 0 || num_splits <= 1) return 0;
    return (size_t)B * H * num_splits * (size_t)(D + 2) * sizeof(float);
}

int hipgpt_attn_decode(const float* q, const float* k, const float* v, float* o, int B, int H, int kv_len, int D,
                       int64_t q_bs, int64_t q_hs, int64_t k_bs, int64_t k_ts, int64_t k_hs, int64_t v_bs,
                       int64_t v_ts, int64_t v_hs, int64_t o_bs, int64_t o_hs, float scale, int num_splits,
                       void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!q || !k || !v || !o || B <= 0 || H <= 0 || kv_len <= 0 || D <= 0 || !std::isfinite(scale))
        return HIPGPT_ERR_INVALID;
    if ((int64_t)B * H > 0x7fffffff) return HIPGPT_ERR_INVALID;
    if (!hipgpt::decode_supported(D, hipgpt::kF32)) return HIPGPT_ERR_UNSUPPORTED;
    const bool ok = aligned16(q) && aligned16(k) && aligned16(v) && q_bs % 4 == 0 && q_hs % 4 == 0 &&
                    k_bs % 4 == 0 && k_ts % 4 == 0 && k_hs % 4 == 0 && v_bs % 4 == 0 && v_ts % 4 == 0 &&
                    v_hs % 4 == 0;
    if (!ok) return HIPGPT_ERR_UNSUPPORTED;
    int ns = num_splits > 0 ? num_splits : hipgpt::decode_default_splits(B, H, kv_len);
    if (ns > kv_len) ns = kv_len;
    const size_t need = hipgpt_attn_decode_workspace_bytes(B, H, D, ns);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return HIPGPT_ERR_WORKSPACE;
    AttnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.q_bs = q_bs;
    a.q_hs = q_hs;
    a.k_bs = k_bs;
    a.k_ts = k_ts;
    a.k_hs = k_hs;
    a.v_bs = v_bs;
    a.v_ts = v_ts;
    a.v_hs = v_hs;
    a.o_bs = o_bs;
    a.o_hs = o_hs;
    a.B = B;
    a.H = H;
    a.Sq = 1;
    a.Sk = kv_len;
    a.D = D;
    a.qscale = default_scale(D, scale) * hipgpt::kLog2e;
    return from_hip(hipgpt::launch_decode(a, hipgpt::kF32, ns, static_cast<float*>(workspace), stream));
}

int hipgpt_attn_decode_kvcache(const float* q, const float* k_new, const float* v_new, float* k_cache,
                               float* v_cache, int* lens, float* o, int B, int H, int D, int max_len, int64_t q_bs,
                               int64_t q_hs, int64_t kn_bs, int64_t kn_hs, int64_t vn_bs, int64_t vn_hs, int64_t c_bs,
                               int64_t c_ts, int64_t c_hs, int64_t o_bs, int64_t o_hs, float scale, int num_splits,
                               int advance, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!q || !k_new || !v_new || !k_cache || !v_cache || !lens || !o || B <= 0 || H <= 0 || D <= 0 ||
        max_len <= 0 || !std::isfinite(scale))
        return HIPGPT_ERR_INVALID;
    if ((int64_t)B * H > 0x7fffffff) return HIPGPT_ERR_INVALID;
    if (!hipgpt::decode_supported(D, hipgpt::kF32)) return HIPGPT_ERR_UNSUPPORTED;
    const bool ok = aligned16(q) && aligned16(k_new) && aligned16(v_new) && aligned16(k_cache) &&
                    aligned16(v_cache) && q_bs % 4 == 0 && q_hs % 4 == 0 && kn_bs % 4 == 0 && kn_hs % 4 == 0 &&
                    vn_bs % 4 == 0 && vn_hs % 4 == 0 && c_bs % 4 == 0 && c_ts % 4 == 0 && c_hs % 4 == 0;
    if (!ok) return HIPGPT_ERR_UNSUPPORTED;
    int ns = num_splits > 0 ? num_splits : hipgpt::decode_default_splits(B, H, max_len);
    if (ns > max_len) ns = max_len;
    const size_t need = hipgpt_attn_decode_workspace_bytes(B, H, D, ns);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return HIPGPT_ERR_WORKSPACE;
    AttnArgs a{};
    a.q = q;
    a.k = k_cache;
    a.v = v_cache;
    a.o = o;
    a.q_bs = q_bs;
    a.q_hs = q_hs;
    a.k_bs = a.v_bs = c_bs;
    a.k_ts = a.v_ts = c_ts;
    a.k_hs = a.v_hs = c_hs;
    a.o_bs = o_bs;
    a.o_hs = o_hs;
    a.B = B;
    a.H = H;
    a.Sq = 1;
    a.Sk = max_len;
    a.D = D;
    a.qscale = default_scale(D, scale) * hipgpt::kLog2e;
    hipgpt::KvcArgs kc{};
    kc.k_new = k_new;
    kc.v_new = v_new;
    kc.kn_bs = kn_bs;
    kc.kn_hs = kn_hs;
    kc.vn_bs = vn_bs;
    kc.vn_hs = vn_hs;
    kc.kc = k_cache;
    kc.vc = v_cache;
    kc.lens = lens;
    kc.max_len = max_len;
    kc.advance = advance ? 1 : 0;
    return from_hip(hipgpt::launch_decode(a, hipgpt::kF32, ns, static_cast<float*>(workspace), stream, &kc));
}

int hipgpt_attn_wait_expired(unsigned int* count, int clear) {
    if (!count) return HIPGPT_ERR_INVALID;
    unsigned int fwd = 0, bwd = 0;
    if (hipgpt::fa_f32_wait_expired(&fwd, clear != 0) != hipSuccess) return HIPGPT_ERR_LAUNCH;
    if (hipgpt::bwd_wait_expired(&bwd, clear != 0) != hipSuccess) return HIPGPT_ERR_LAUNCH;
    *count = fwd + bwd;
    return HIPGPT_OK;
}

void hipgpt_launch_matmul(const float* A, const float* B, float* C, int M, int N, int K) {
    launch_matmul(A, B, C, M, N, K);
}

void hipgpt_launch_matmul_add_bias(const float* A, const float* B, const float* bias, float* C, int M, int N,
                                   int K) {
    launch_matmul_add_bias(A, B, bias, C, M, N, K);
}

int hipgpt_gemm_bias(const float* A, const float* W, const float* bias, void* C, int M, int N, int K, int64_t lda,
                     int64_t ldw, int64_t ldc, int seg_w, int64_t seg_stride, int out_dtype, hipStream_t stream) {
    if (!C || M <= 0 || N <= 0 || K < 0 || (K > 0 && (!A || !W))) return HIPGPT_ERR_INVALID;
    if (lda < K || ldw < N || seg_w < 1 || seg_w > N || ldc < seg_w || seg_stride < 0) return HIPGPT_ERR_INVALID;
    if (out_dtype != HIPGPT_F32 && out_dtype != HIPGPT_BF16) return HIPGPT_ERR_INVALID;
    hipgpt::GemmArgs g{};
    g.A = A;
    g.W = W;
    g.bias = bias;
    g.C = C;
    g.M = M;
    g.N = N;
    g.K = K;
    g.lda = lda;
    g.ldw = ldw;
    g.ldc = ldc;
    g.seg_w = seg_w;
    g.seg_stride = seg_stride;
    g.out_bf16 = out_dtype == HIPGPT_BF16;
    return from_hip(hipgpt::launch_gemm(g, stream));
}

int hipgpt_qkv_projection(const float* x, const float* w_qkv, const float* b_qkv, void* out, int T, int E, int layout,
                          int out_dtype, hipStream_t stream) {
    if (T <= 0 || E <= 0 || (int64_t)3 * E > 0x7fffffff) return HIPGPT_ERR_INVALID;
    if (layout != HIPGPT_QKV_ROWS && layout != HIPGPT_QKV_PLANAR) return HIPGPT_ERR_INVALID;
    const int N = 3 * E;
    if (layout == HIPGPT_QKV_ROWS)
        return hipgpt_gemm_bias(x, w_qkv, b_qkv, out, T, N, E, E, N, N, N, 0, out_dtype, stream);
    return hipgpt_gemm_bias(x, w_qkv, b_qkv, out, T, N, E, E, N, E, E, (int64_t)T * E, out_dtype, stream);
}

}  // extern "C"
