// helpers.hip -- HipGPT's unfused single-head attention helpers.
//
// Replaces scaled_dot_product_kernel, softmax_kernel and
// attention_weighted_sum_kernel (HipGPT src/hip_kernels.cpp:454-532, declared
// include/hip_kernels.h:44-46).  HipGPT itself no longer calls them (the
// flash path replaced them), but they are part of the header a drop-in must
// provide.  Layouts: Q, K, V, O are [B*S][D]; scores / probs are [B*S][S];
// non-causal.
//   * scores = Q K^T * rsqrt(D): one wave per 32x32 tile on
//     v_mfma_f32_32x32x2_f32, operands straight from global memory (each K
//     row is read by the S/32 query tiles of its batch through L2), scale
//     applied to the fp32 accumulator as the reference does.
//   * row softmax: one wave per row, wave max / wave sum, exp2 on the
//     transcendental unit; HBM-bound.
//   * out = P V: O^T = V^T P^T per (32-query tile, 32-column block) wave;
//     P^T is read in the accumulator's key order (four float4 per 32 keys).
// Head dims above 128 use a scalar kernel (one thread per output element).
#include "common.h"
#include "fa_common.h"
#include "kernels.h"

namespace hipgpt {

namespace {

using fa::acc_key;

// ---------------------------------------------------------------- Q K^T
template <int DP>
__global__ __launch_bounds__(256) void sdp_mfma_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                                                       float* __restrict__ scores, int B, int S, int D, float inv) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 31, hf = lane >> 5;
    const int nt = (S + 31) / 32;
    const int qt = blockIdx.x, b = blockIdx.y;
    const int qi = qt * 32 + c;
    const float* Qb = Q + (int64_t)b * S * D;
    const float* Kb = K + (int64_t)b * S * D;
    // B operand: lane (c, hf) holds Q[qi][hf*DP/2 + s]
    float qf[DP / 2];
#pragma unroll
    for (int s = 0; s < DP / 2; ++s) {
        const int d = hf * (DP / 2) + s;
        qf[s] = (qi < S && d < D) ? Qb[(int64_t)qi * D + d] : 0.f;
    }
    for (int kt = wave; kt < nt; kt += 4) {
        const int key = kt * 32 + c;
        floatx16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
        for (int s = 0; s < DP / 2; ++s) {
            const int d = hf * (DP / 2) + s;
            const float kv = (key < S && d < D) ? Kb[(int64_t)key * D + d] : 0.f;
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv, qf[s], acc, 0, 0, 0);
        }
        if (qi < S) {
            float* row = scores + ((int64_t)b * S + qi) * S;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = kt * 32 + acc_key(r, hf);
                if (j < S) row[j] = acc[r] * inv;
            }
        }
    }
}

__global__ __launch_bounds__(256) void sdp_scalar_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                                                         float* __restrict__ scores, int B, int S, int D, float inv) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = (int64_t)B * S * S;
    if (idx >= n) return;
    const int64_t tok = idx / S;
    const int j = (int)(idx % S);
    const float* q = Q + tok * D;
    const float* k = K + ((tok / S) * S + j) * (int64_t)D;
    float acc = 0.f;
    for (int d = 0; d < D; ++d) acc = fmaf(q[d], k[d], acc);
    scores[idx] = acc * inv;
}

// ---------------------------------------------------------------- softmax
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                           int64_t rows, int S) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* x = in + row * S;
    float* y = out + row * S;
    float m = kMaxInit;
    for (int j = lane; j < S; j += 64) m = fmaxf(m, x[j]);
    m = wave_max(m);
    float s = 0.f;
    for (int j = lane; j < S; j += 64) {
        const float e = fast_exp2((x[j] - m) * kLog2e);
        y[j] = e;
        s += e;
    }
    const float inv = 1.0f / fmaxf(wave_sum(s), 1e-20f);
    for (int j = lane; j < S; j += 64) y[j] *= inv;
}

// ---------------------------------------------------------------- P V
// One wave per (32-query tile, 32-column block of O).
__global__ __launch_bounds__(64) void wsum_mfma_kernel(const float* __restrict__ P, const float* __restrict__ V,
                                                       float* __restrict__ O, int B, int S, int D) {
    const int lane = threadIdx.x, c = lane & 31, hf = lane >> 5;
    const int qt = blockIdx.x, db = blockIdx.y, b = blockIdx.z;
    const int qi = qt * 32 + c;
    const int dcol = db * 32 + c;
    const float* Pr = P + ((int64_t)b * S + qi) * S;
    const float* Vb = V + (int64_t)b * S * D;
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    for (int kt = 0; kt * 32 < S; ++kt) {
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int j = kt * 32 + acc_key(t, hf);
            const float p = (qi < S && j < S) ? Pr[j] : 0.f;                       // B: P^T[j][qi]
            const float v = (j < S && dcol < D) ? Vb[(int64_t)j * D + dcol] : 0.f;  // A: V^T[dcol][j]
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(v, p, acc, 0, 0, 0);
        }
    }
    if (qi < S) {
        float* orow = O + ((int64_t)b * S + qi) * D;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int d = db * 32 + acc_key(r, hf);
            if (d < D) orow[d] = acc[r];
        }
    }
}

}  // namespace

hipError_t launch_sdp(const float* Q, const float* K, float* scores, int B, int S, int D, hipStream_t s) {
    const float inv = 1.0f / sqrtf((float)D);
    const int nt = (S + 31) / 32;
    if (D <= 128) {
        dim3 grid(nt, B);
        if (D <= 32)
            hipLaunchKernelGGL(sdp_mfma_kernel<32>, grid, dim3(256), 0, s, Q, K, scores, B, S, D, inv);
        else if (D <= 64)
            hipLaunchKernelGGL(sdp_mfma_kernel<64>, grid, dim3(256), 0, s, Q, K, scores, B, S, D, inv);
        else
            hipLaunchKernelGGL(sdp_mfma_kernel<128>, grid, dim3(256), 0, s, Q, K, scores, B, S, D, inv);
    } else {
        const int64_t n = (int64_t)B * S * S;
        const int64_t blocks = (n + 255) / 256;
        if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
        hipLaunchKernelGGL(sdp_scalar_kernel, dim3((unsigned)blocks), dim3(256), 0, s, Q, K, scores, B, S, D, inv);
    }
    return hipGetLastError();
}

hipError_t launch_softmax_rows(const float* in, float* out, int B, int S, hipStream_t s) {
    const int64_t rows = (int64_t)B * S;
    const int64_t blocks = (rows + 3) / 4;
    if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, s, in, out, rows, S);
    return hipGetLastError();
}

hipError_t launch_wsum(const float* P, const float* V, float* O, int B, int S, int D, hipStream_t s) {
    dim3 grid((S + 31) / 32, (D + 31) / 32, B);
    hipLaunchKernelGGL(wsum_mfma_kernel, grid, dim3(64), 0, s, P, V, O, B, S, D);
    return hipGetLastError();
}

}  // namespace hipgpt
