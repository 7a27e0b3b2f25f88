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
//
// KV-cache mode (KVC): K/V are a cache [B][max_len][H][D] with a device
// length lens[b] per sequence; the step's own key/value row (k_new, v_new)
// sits at position lens[b].  Splits cover the lens[b] + 1 visible keys of
// their sequence; the split that owns position lens[b] takes that row from
// k_new / v_new and writes it into the cache (no other workgroup touches
// that cache row, so there is no race).  A sequence whose length is outside
// [0, max_len) is left untouched and its output is NaN (the partial sum is
// poisoned, so the reduce propagates it).  lens[b] is advanced by the reduce
// kernel's workgroup for head 0 -- reduce workgroups never read lens -- or,
// with one split, by a one-thread-per-sequence kernel after the step.
#include "common.h"
#include "kernels.h"

namespace hipgpt {

namespace {

constexpr int DEC_NW = 4;  // waves per workgroup

template <int DP, int U, bool KVC>
__global__ __launch_bounds__(DEC_NW * 64) void decode_partial_kernel(AttnArgs a, KvcArgs kc, int nsplit, int chunk,
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
    int k0 = split * chunk;
    int k1 = min(a.Sk, k0 + chunk);
    int len = 0;        // KVC: cached rows before the new one
    bool bad = false;   // KVC: length outside [0, max_len)
    bool owns_new = false;
    if (KVC) {
        len = kc.lens[b];
        bad = len < 0 || len >= kc.max_len;
        const int kv = bad ? 0 : len + 1;
        const int ch = (kv + nsplit - 1) / nsplit;
        k0 = split * ch;
        k1 = min(kv, k0 + ch);
        owns_new = k0 <= len && len < k1;
        if (owns_new) k1 = len;  // cache rows only; the new row is added below
    }

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

    if (KVC && owns_new) {
        // the step's own key/value row: into the online softmax of group 0
        // of wave 0 (lanes 0..LPK-1) and into the cache at position len
        const float* kn = kc.k_new + b * kc.kn_bs + h * kc.kn_hs + sub * 4;
        const float* vn = kc.v_new + b * kc.vn_bs + h * kc.vn_hs + sub * 4;
        floatx4 kv4 = {0.f, 0.f, 0.f, 0.f}, vv4 = {0.f, 0.f, 0.f, 0.f};
        if (tid < LPK) {
            kv4 = *reinterpret_cast<const floatx4*>(kn);
            vv4 = *reinterpret_cast<const floatx4*>(vn);
            *reinterpret_cast<floatx4*>(kc.kc + b * a.k_bs + (int64_t)len * a.k_ts + h * a.k_hs + sub * 4) = kv4;
            *reinterpret_cast<floatx4*>(kc.vc + b * a.v_bs + (int64_t)len * a.v_ts + h * a.v_hs + sub * 4) = vv4;
        }
        float d = q4[0] * kv4[0];
        d = fmaf(q4[1], kv4[1], d);
        d = fmaf(q4[2], kv4[2], d);
        d = fmaf(q4[3], kv4[3], d);
#pragma unroll
        for (int msk = LPK / 2; msk >= 1; msk >>= 1) d += __shfl_xor(d, msk);
        if (slot == 0) {
            const float m_new = fmaxf(m, d);
            const float alpha = fast_exp2(m - m_new);
            const float p = fast_exp2(d - m_new);
            l = fmaf(l, alpha, p);
            o4 = o4 * alpha + p * vv4;
            m = m_new;
        }
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
        if (KVC && bad) L = O = __builtin_nanf("");  // poisons this (b, h): output NaN
        if (nsplit == 1) {
            if (d < a.D) a.o[b * a.o_bs + h * a.o_hs + d] = KVC && bad ? O : O / fmaxf(L, 1e-20f);
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

// Merge of the splits of one (b, h) row, with the splits in parallel: the
// (m, l) pairs are reduced by all 256 threads (block max, then block sum of
// l_s 2^(m_s - M)); the O rows by DP/4 lanes per split row (one float4 each)
// and 1024/DP split rows at a time, combined through LDS.
constexpr int RED_T = 256;

template <int DP>
__global__ __launch_bounds__(RED_T) void decode_reduce_kernel(AttnArgs a, int nsplit, const float* ws,
                                                              int* advance_lens, int max_len) {
    constexpr int LP = DP / 4;         // lanes per split row
    constexpr int SG = RED_T / LP;     // split rows in flight
    __shared__ float red[RED_T / 64];
    __shared__ __attribute__((aligned(16))) float s_o[SG][DP];
    const int bh = blockIdx.x;
    const int BH = a.B * a.H;
    const int b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // KV-cache step: the head-0 workgroup advances its sequence (no reduce
    // workgroup reads lens, and the partial kernel has completed)
    if (advance_lens && h == 0 && tid == 0) {
        const int n = advance_lens[b];
        if (n >= 0 && n < max_len) advance_lens[b] = n + 1;
    }
    const float* wml = ws + (int64_t)bh * nsplit * 2;
    const float* wo = ws + (int64_t)BH * nsplit * 2 + (int64_t)bh * nsplit * DP;

    float mx = kMaxInit;
    for (int s = tid; s < nsplit; s += RED_T) mx = fmaxf(mx, wml[2 * s]);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < RED_T / 64; ++w) M = fmaxf(M, red[w]);
    __syncthreads();
    float ls = 0.f;
    for (int s = tid; s < nsplit; s += RED_T) ls = fmaf(wml[2 * s + 1], fast_exp2(wml[2 * s] - M), ls);
    ls = wave_sum(ls);
    if (lane == 0) red[wave] = ls;
    __syncthreads();
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < RED_T / 64; ++w) L += red[w];

    const int sub = tid % LP, sg = tid / LP;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int s = sg; s < nsplit; s += SG) {
        const float w = fast_exp2(wml[2 * s] - M);
        acc += w * *reinterpret_cast<const floatx4*>(wo + (int64_t)s * DP + sub * 4);
    }
    *reinterpret_cast<floatx4*>(&s_o[sg][sub * 4]) = acc;
    __syncthreads();
    const float linv = 1.0f / fmaxf(L, 1e-20f);
    for (int d = tid; d < a.D; d += RED_T) {
        float O = 0.f;
#pragma unroll
        for (int g = 0; g < SG; ++g) O += s_o[g][d];
        a.o[b * a.o_bs + h * a.o_hs + d] = O * linv;
    }
}

__global__ __launch_bounds__(256) void kvc_advance_kernel(int* lens, int B, int max_len) {
    const int b = blockIdx.x * 256 + threadIdx.x;
    if (b < B) {
        const int n = lens[b];
        if (n >= 0 && n < max_len) lens[b] = n + 1;
    }
}

int decode_padded_dim(int D) {
    if (D == 32 || D == 64 || D == 128 || D == 256) return D;
    return 0;
}

template <int DP>
hipError_t launch_decode_dp(const AttnArgs& a, const KvcArgs* kc, int nsplit, float* ws, hipStream_t stream) {
    constexpr int U = DP >= 128 ? 4 : 8;
    const int BH = a.B * a.H;
    const int chunk = (a.Sk + nsplit - 1) / nsplit;
    const int64_t grid = (int64_t)BH * nsplit;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    if (kc)
        hipLaunchKernelGGL((decode_partial_kernel<DP, U, true>), dim3((unsigned)grid), dim3(DEC_NW * 64), 0, stream, a,
                           *kc, nsplit, chunk, ws);
    else
        hipLaunchKernelGGL((decode_partial_kernel<DP, U, false>), dim3((unsigned)grid), dim3(DEC_NW * 64), 0, stream,
                           a, KvcArgs{}, nsplit, chunk, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    int* adv = kc && kc->advance ? kc->lens : nullptr;
    const int max_len = kc ? kc->max_len : 0;
    if (nsplit > 1) {
        hipLaunchKernelGGL((decode_reduce_kernel<DP>), dim3((unsigned)BH), dim3(RED_T), 0, stream, a, nsplit,
                           static_cast<const float*>(ws), adv, max_len);
        e = hipGetLastError();
    } else if (adv) {
        hipLaunchKernelGGL(kvc_advance_kernel, dim3((unsigned)((a.B + 255) / 256)), dim3(256), 0, stream, adv, a.B,
                           max_len);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace

bool decode_supported(int D, int dtype) { return dtype == kF32 && decode_padded_dim(D) != 0; }

// Split only until there are more than 512 workgroups (2+ per CU): each
// split adds partial writes and the reduce launch, and with B*H above 512 one
// split per (b, h) streams fastest (c5: 124.6 us at 1 split, 129 us at 4).
// No split shorter than 128 keys.
int decode_default_splits(int B, int H, int kv_len) {
    const int64_t bh = (int64_t)B * H;
    int n = 1;
    while (n < 64 && bh * n <= 512 && (int64_t)kv_len / (2 * n) >= 128) n *= 2;
    return n;
}

hipError_t launch_decode(const AttnArgs& a, int dtype, int nsplit, float* ws, hipStream_t stream,
                         const KvcArgs* kc) {
    if (!decode_supported(a.D, dtype) || nsplit < 1) return hipErrorInvalidValue;
    if (nsplit > 1 && ws == nullptr) return hipErrorInvalidValue;
    switch (decode_padded_dim(a.D)) {
        case 32: return launch_decode_dp<32>(a, kc, nsplit, ws, stream);
        case 64: return launch_decode_dp<64>(a, kc, nsplit, ws, stream);
        case 128: return launch_decode_dp<128>(a, kc, nsplit, ws, stream);
        case 256: return launch_decode_dp<256>(a, kc, nsplit, ws, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hipgpt
