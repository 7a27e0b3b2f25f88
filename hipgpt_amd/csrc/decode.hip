// decode.hip -- split-KV attention for one new query row per sequence.
//
// No reference kernel exists: HipGPT's generate loop recomputes the whole
// window (src/gpt_model.cpp:261-273), so a decode step's output is the last
// row of full attention over the kv_len keys (src/hip_kernels.cpp:329-402
// at S = kv_len).  This is the kernel a KV-cached loop would call.
//
// The shape is HBM-bound (every K/V byte is read once, ~0.5 flop/byte), so
// it runs on the vector ALUs, not MFMA:
//   * partial kernel: one workgroup per (batch*head, split).  A key row of
//     D floats is covered by D/4 lanes (one float4 each), so a wave reads
//     64/(D/4) whole rows per load; U loads per lane are in flight at once.
//     q.k is a DPP/shuffle reduction inside the D/4-lane group; each group
//     keeps its own online-softmax state (m, l, O slice); the groups are
//     merged through LDS at the end.  With one split the result is final.
//   * reduce kernel: merges the splits' (m, l, O) with the log-sum-exp rule
//       M = max m_s,  L = sum l_s 2^(m_s - M),  O = sum O_s 2^(m_s - M) / L.
#include "common.h"
#include "kernels.h"

namespace hipgpt {

namespace {

constexpr int DEC_NW = 4;  // waves per workgroup

template <int DP, int U>
__global__ __launch_bounds__(DEC_NW * 64) void decode_partial_kernel(AttnArgs a, int nsplit, int chunk,
                                                                     float* ws) {
    constexpr int LPK = DP / 4;   // lanes per key row
    constexpr int KPW = 64 / LPK; // key rows per wave per load
    constexpr int G = DEC_NW * KPW;  // key rows per workgroup per load
    __shared__ float s_ml[G][2];
    __shared__ __attribute__((aligned(16))) float s_o[G][DP];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int grp = lane / LPK;   // key group inside the wave
    const int sub = lane % LPK;   // float4 column of the row
    const int slot = wave * KPW + grp;

    const int BH = a.B * a.H;
    const int bh = blockIdx.x % BH;
    const int split = blockIdx.x / BH;
    const int b = bh / a.H, h = bh % a.H;
    const int k0 = split * chunk;
    const int k1 = min(a.Sk, k0 + chunk);

    const float* qp = static_cast<const float*>(a.q) + b * a.q_bs + h * a.q_hs;
    const float* Kp = static_cast<const float*>(a.k) + b * a.k_bs + h * a.k_hs + sub * 4;
    const float* Vp = static_cast<const float*>(a.v) + b * a.v_bs + h * a.v_hs + sub * 4;

    floatx4 q4 = *reinterpret_cast<const floatx4*>(qp + sub * 4);
    q4 *= a.qscale;

    float m = kMaxInit, l = 0.f;
    floatx4 o4 = {0.f, 0.f, 0.f, 0.f};

    for (int kb = k0 + slot; kb < k1; kb += G * U) {
        floatx4 kv[U], vv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int key = kb + u * G;
            if (key < k1) {
                kv[u] = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(Kp + (int64_t)key * a.k_ts));
                vv[u] = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(Vp + (int64_t)key * a.v_ts));
            } else {
                kv[u] = floatx4{0.f, 0.f, 0.f, 0.f};
                vv[u] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
        }
        float s[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float d = q4[0] * kv[u][0];
            d = fmaf(q4[1], kv[u][1], d);
            d = fmaf(q4[2], kv[u][2], d);
            d = fmaf(q4[3], kv[u][3], d);
#pragma unroll
            for (int msk = LPK / 2; msk >= 1; msk >>= 1) d += __shfl_xor(d, msk);
            s[u] = (kb + u * G < k1) ? d : kNegInf;
        }
        float mt = s[0];
#pragma unroll
        for (int u = 1; u < U; ++u) mt = fmaxf(mt, s[u]);
        const float m_new = fmaxf(m, mt);
        const float alpha = fast_exp2(m - m_new);
        l *= alpha;
        o4 *= alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float p = fast_exp2(s[u] - m_new);
            l += p;
            o4[0] = fmaf(p, vv[u][0], o4[0]);
            o4[1] = fmaf(p, vv[u][1], o4[1]);
            o4[2] = fmaf(p, vv[u][2], o4[2]);
            o4[3] = fmaf(p, vv[u][3], o4[3]);
        }
        m = m_new;
    }

    if (sub == 0) {
        s_ml[slot][0] = m;
        s_ml[slot][1] = l;
    }
    *reinterpret_cast<floatx4*>(&s_o[slot][sub * 4]) = o4;
    __syncthreads();

    if (tid < DP) {
        const int d = tid;
        float M = kMaxInit;
#pragma unroll
        for (int g = 0; g < G; ++g) M = fmaxf(M, s_ml[g][0]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float w = fast_exp2(s_ml[g][0] - M);
            L = fmaf(s_ml[g][1], w, L);
            O = fmaf(s_o[g][d], w, O);
        }
        if (nsplit == 1) {
            if (d < a.D) a.o[b * a.o_bs + h * a.o_hs + d] = O / fmaxf(L, 1e-20f);
        } else {
            float* wml = ws + ((int64_t)bh * nsplit + split) * 2;
            float* wo = ws + (int64_t)BH * nsplit * 2 + ((int64_t)bh * nsplit + split) * DP;
            if (d == 0) {
                wml[0] = M;
                wml[1] = L;
            }
            wo[d] = O;
        }
    }
}

template <int DP>
__global__ __launch_bounds__(64) void decode_reduce_kernel(AttnArgs a, int nsplit, const float* ws) {
    const int bh = blockIdx.x;
    const int BH = a.B * a.H;
    const int b = bh / a.H, h = bh % a.H;
    const float* wml = ws + (int64_t)bh * nsplit * 2;
    const float* wo = ws + (int64_t)BH * nsplit * 2 + (int64_t)bh * nsplit * DP;
    float M = kMaxInit;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, wml[2 * s]);
    float L = 0.f;
    for (int s = 0; s < nsplit; ++s) L = fmaf(wml[2 * s + 1], fast_exp2(wml[2 * s] - M), L);
    const float linv = 1.0f / fmaxf(L, 1e-20f);
    for (int d = threadIdx.x; d < a.D; d += 64) {
        float O = 0.f;
        for (int s = 0; s < nsplit; ++s) O = fmaf(wo[(int64_t)s * DP + d], fast_exp2(wml[2 * s] - M), O);
        a.o[b * a.o_bs + h * a.o_hs + d] = O * linv;
    }
}

int decode_padded_dim(int D) {
    if (D == 32 || D == 64 || D == 128 || D == 256) return D;
    return 0;
}

template <int DP>
hipError_t launch_decode_dp(const AttnArgs& a, int nsplit, float* ws, hipStream_t stream) {
    constexpr int U = DP >= 128 ? 4 : 8;
    const int BH = a.B * a.H;
    const int chunk = (a.Sk + nsplit - 1) / nsplit;
    const int64_t grid = (int64_t)BH * nsplit;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((decode_partial_kernel<DP, U>), dim3((unsigned)grid), dim3(DEC_NW * 64), 0, stream, a,
                       nsplit, chunk, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || nsplit == 1) return e;
    hipLaunchKernelGGL((decode_reduce_kernel<DP>), dim3((unsigned)BH), dim3(64), 0, stream, a, nsplit,
                       static_cast<const float*>(ws));
    return hipGetLastError();
}

}  // namespace

bool decode_supported(int D, int dtype) { return dtype == kF32 && decode_padded_dim(D) != 0; }

// Enough workgroups to cover the chip several times over, but no split
// shorter than 128 keys.
int decode_default_splits(int B, int H, int kv_len) {
    const int64_t bh = (int64_t)B * H;
    int n = 1;
    while (n < 64 && bh * n < 2048 && (int64_t)kv_len / (2 * n) >= 128) n *= 2;
    return n;
}

hipError_t launch_decode(const AttnArgs& a, int dtype, int nsplit, float* ws, hipStream_t stream) {
    if (!decode_supported(a.D, dtype) || nsplit < 1) return hipErrorInvalidValue;
    if (nsplit > 1 && ws == nullptr) return hipErrorInvalidValue;
    switch (decode_padded_dim(a.D)) {
        case 32: return launch_decode_dp<32>(a, nsplit, ws, stream);
        case 64: return launch_decode_dp<64>(a, nsplit, ws, stream);
        case 128: return launch_decode_dp<128>(a, nsplit, ws, stream);
        case 256: return launch_decode_dp<256>(a, nsplit, ws, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hipgpt
