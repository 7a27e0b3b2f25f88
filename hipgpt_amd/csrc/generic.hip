// generic.hip -- fp32 attention forward for any head dim (the path the MFMA
// kernel does not cover: D > 128, or problems the caller wants bit-simple).
//
// Serves the part of multihead_attention_kernel_fallback's domain
// (HipGPT src/hip_kernels.cpp:329-402, any D = E/H) outside the MFMA
// specialisations.  One wave per query row:
//   sweep A: 64 keys at a time, one key per lane (full-D dot product per
//            lane), wave max / wave sum give the row max m and sum l;
//   sweep B: recompute the scores, p = exp(s - m) / l (stored to probs when
//            requested), broadcast p lane by lane and accumulate O with the
//            lanes spread over d (64*GC columns per pass; larger D takes
//            several passes, each recomputing the scores).
#include "common.h"
#include "kernels.h"

namespace hipgpt {

namespace {

constexpr int GC = 8;  // d columns per lane per pass (512 per pass)

template <bool CAUSAL>
__global__ __launch_bounds__(256) void attn_generic_f32_kernel(AttnArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t nrows = (int64_t)a.B * a.H * a.Sq;
    if (row >= nrows) return;  // wave-uniform
    const int i = (int)(row % a.Sq);
    const int bh = (int)(row / a.Sq);
    const int b = bh / a.H, h = bh % a.H;
    const int D = a.D, Sk = a.Sk;
    const int nvis = CAUSAL ? min(Sk, i + 1 + a.causal_off) : Sk;

    const float* q = static_cast<const float*>(a.q) + b * a.q_bs + h * a.q_hs + (int64_t)i * a.q_ts;
    const float* K = static_cast<const float*>(a.k) + b * a.k_bs + h * a.k_hs;
    const float* V = static_cast<const float*>(a.v) + b * a.v_bs + h * a.v_hs;
    float* o = a.o + b * a.o_bs + h * a.o_hs + (int64_t)i * a.o_ts;
    float* prow = a.probs ? a.probs + ((int64_t)bh * a.Sq + i) * (int64_t)Sk : nullptr;

    auto score = [&](int j) -> float {
        if (j >= nvis) return kNegInf;
        const float* k = K + (int64_t)j * a.k_ts;
        float acc = 0.f;
        for (int d = 0; d < D; ++d) acc = fmaf(q[d], k[d], acc);
        return acc * a.qscale;
    };

    float m = kMaxInit, l = 0.f;
    for (int jt = 0; jt < nvis; jt += 64) {
        const float s = score(jt + lane);
        const float m_new = fmaxf(m, wave_max(s));
        l = l * fast_exp2(m - m_new) + wave_sum(fast_exp2(s - m_new));
        m = m_new;
    }
    const float linv = 1.0f / fmaxf(l, 1e-20f);

    for (int dc = 0; dc < D; dc += 64 * GC) {
        float acc[GC];
#pragma unroll
        for (int g = 0; g < GC; ++g) acc[g] = 0.f;
        for (int jt = 0; jt < nvis; jt += 64) {
            const int j = jt + lane;
            const float p = fast_exp2(score(j) - m) * linv;  // 0 for j >= nvis
            if (prow && dc == 0 && j < nvis) prow[j] = p;
            const int nj = min(64, nvis - jt);
            for (int jj = 0; jj < nj; ++jj) {
                const float pj = __shfl(p, jj);
                const float* v = V + (int64_t)(jt + jj) * a.v_ts;
#pragma unroll
                for (int g = 0; g < GC; ++g) {
                    const int d = dc + lane + 64 * g;
                    if (d < D) acc[g] = fmaf(pj, v[d], acc[g]);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < GC; ++g) {
            const int d = dc + lane + 64 * g;
            if (d < D) o[d] = acc[g];
        }
    }
    if (prow)
        for (int j = nvis + lane; j < Sk; j += 64) prow[j] = 0.f;
}

}  // namespace

hipError_t launch_attn_generic_f32(const AttnArgs& a, bool causal, hipStream_t stream) {
    const int64_t rows = (int64_t)a.B * a.H * a.Sq;
    const int64_t grid = (rows + 3) / 4;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    if (causal)
        hipLaunchKernelGGL(attn_generic_f32_kernel<true>, dim3((unsigned)grid), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(attn_generic_f32_kernel<false>, dim3((unsigned)grid), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace hipgpt
