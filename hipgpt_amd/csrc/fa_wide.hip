// fa_wide.hip -- fp32 attention forward on gfx950 MFMA for head dims above
// 128 (128 < D <= 512, D % 4 == 0, 16-byte aligned rows; padded to 256 or 512).
//
// Replaces, for those head dims, multihead_attention_kernel_fallback (HipGPT
// src/hip_kernels.cpp:329-402), the reference's path for any head dim other
// than 32 and 64.  The per-wave kernel of fa_kernel.h holds a wave's 32 query
// rows of Q and of the O accumulator in registers, D/2 + D/2 values per lane,
// which stops fitting above D = 128.  Here the head dim is split instead:
//   * the DH waves of a query sub-block (4 at padded D = 256, 8 at 512) share
//     its 32 queries and each holds 64 of the head dims of Q (pre-scaled by
//     scale*log2 e) and of the O accumulator;
//   * per key tile, each wave forms its partial S^T = K Q^T over its dims,
//     the DH partials go through LDS and every wave adds them in the same
//     order, so all of them hold the same scores bit for bit and run the same
//     online softmax (lazy rescale, as fa_kernel.h); then each wave
//     accumulates O^T += V^T P^T for its own dims.
// K and V tiles are row-major in LDS (rowtiles.h) in one stage buffer: the
// next stage waits in registers during the MFMAs and is stored after a
// barrier (two buffers would not fit next to the partial-score exchange).  At
// padded D = 512 one K and one V tile do not fit together either: the V tile
// of key tile t is requested during its scores and stored over the K tile
// once every wave has read it, and K of tile t+1 is requested during P V.
// With probs (the drop-in contract): sweep 1 forms each row's max and sum
// (K tiles only); sweep 2 recomputes the scores, stores P = exp2(s' - m -
// log2 l) -- every element by exactly one of the DH waves -- and accumulates
// P V.  Causal: key tiles past a sub-block's diagonal are skipped,
// the diagonal tiles masked, and the probs above the diagonal stored as 0.
#include "common.h"
#include "fa_common.h"
#include "kernels.h"
#include "rowtiles.h"

namespace hipgpt {

namespace {

using fa::acc_key;
using fa::kLazyMax;
using fa::QW;

template <int DP, int DH, int NQB, bool CAUSAL, bool PROBS>
struct WideFwd {
    using T = RowTiles<DP, DH>;
    static_assert(DH == 4 || DH == 8, "probs stores split over 4 or 8 waves");
    static constexpr bool SPLIT = DP > 256;  // K and V tiles take turns in the stage buffer
    static constexpr int NW = NQB * DH;
    static constexpr int NT = NW * 64;
    static constexpr int STAGE = (SPLIT ? 1 : 2) * T::ROW;  // K (, V) row-major
    static constexpr int XCH = NW * 16 * 64;                 // partial score tiles
    static constexpr int LDS_FLOATS = STAGE + XCH;

    __device__ __forceinline__ static void run(const AttnArgs& a, float* lds) {
        const int tid = threadIdx.x, lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int c = lane & 31, hf = lane >> 5;
        const int sb = wave / DH, dh = wave % DH;
        const int BH = a.B * a.H;
        const int bh = blockIdx.x % BH;
        const int rank = blockIdx.x / BH;
        const int qb = CAUSAL ? a.n_qblk - 1 - rank : rank;  // longest rows first
        const int b = bh / a.H, h = bh % a.H;
        const int q0 = qb * NQB * QW, qw0 = q0 + sb * QW, qi = qw0 + c;
        const int Sq = a.Sq, Sk = a.Sk, off = a.causal_off, D = a.D;
        const float* Qp = static_cast<const float*>(a.q) + b * a.q_bs + h * a.q_hs;
        const float* Kp = static_cast<const float*>(a.k) + b * a.k_bs + h * a.k_hs;
        const float* Vp = static_cast<const float*>(a.v) + b * a.v_bs + h * a.v_hs;
        const fa::TileRange tr = fa::tile_range<CAUSAL>(q0, qw0, NQB * QW, Sq, Sk, off);
        const int nstages = tr.ntiles, wtiles = tr.wtiles;

        float q[T::DW / 2];  // B operand of S^T = K Q^T: Q[qi][wave's dims] * scale * log2 e
        {
            const int d0 = dh * T::DW + hf * (T::DW / 2);
            const float* p = Qp + (int64_t)qi * a.q_ts + d0;
#pragma unroll
            for (int s = 0; s < T::DW / 2; s += 4) {
                const floatx4 t = (qi < Sq && d0 + s < D) ? *reinterpret_cast<const floatx4*>(p + s)
                                                          : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) q[s + j] = t[j] * a.qscale;
            }
        }
        RowLoader kl, vl;
        kl.init(Kp, a.k_ts, Sk, D);
        vl.init(Vp, a.v_ts, Sk, D);
        floatx4* const xch = reinterpret_cast<floatx4*>(lds + STAGE);

        floatx16 o[1][T::NDBW];  // O^T: [d][query]
#pragma unroll
        for (int db = 0; db < T::NDBW; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[0][db][r] = 0.f;
        float m_run = kMaxInit, l_run = 0.f;

        // Scores of tile t (log2 units, masked), the same bits in all DH
        // waves of the sub-block; every wave of the workgroup calls it (one
        // barrier inside).
        auto scores = [&](bool act, int t) -> floatx16 {
            floatx16 s;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = 0.f;
            if (act) {
                T::dchain(s, lds, q, c, hf, dh);
                T::publish(s, xch, wave, lane);
            }
            __syncthreads();
            if (act) {
                s = T::total(s, xch, sb, dh, lane);
                if (tr.edge(t, Sk, CAUSAL, qw0, off)) fa::mask_tile<CAUSAL>(s, t * BK, hf, qi, Sk, off);
            }
            return s;
        };

        // MODE 0: online softmax + P V.  1: row max / sum only (K staged
        // alone).  2: probs stored with the final (m, l) + P V.
        auto sweep = [&](auto mode_tag, float mlog, float* prow, bool pvec) {
            constexpr int MODE = decltype(mode_tag)::value;
            constexpr bool TURNS = SPLIT && MODE != 1;  // V takes K's place after the scores
            RowStage<DP, NT, (SPLIT || MODE == 1) ? 1 : 2> stg;
            const float* const vt = lds + (SPLIT ? 0 : T::ROW);
            if (nstages > 0) {
                stg.load(kl, vl, 0, D, tid);
                stg.store(lds, T::ROW, tid);
            }
            __syncthreads();
            for (int t = 0; t < nstages; ++t) {
                if constexpr (TURNS)
                    stg.load(vl, vl, t * BK, D, tid);  // V of this tile, in flight during its scores
                else if (t + 1 < nstages)
                    stg.load(kl, vl, (t + 1) * BK, D, tid);
                const bool act = t < wtiles;  // wave-uniform
                floatx16 s = scores(act, t);   // past its barrier no wave reads this K tile again
                if constexpr (TURNS) {
                    stg.store(lds, T::ROW, tid);
                    __syncthreads();
                    if (t + 1 < nstages) stg.load(kl, vl, (t + 1) * BK, D, tid);  // next K, during P V
                }
                if (act) {
                    if constexpr (MODE == 0) {
                        const float tmax = fa::tile_max(s);
                        if (__any(tmax > m_run + kLazyMax)) {
                            const float m_new = fa::vmax(m_run, tmax);
                            const float alpha = fast_exp2(m_run - m_new);
                            l_run *= alpha;
#pragma unroll
                            for (int db = 0; db < T::NDBW; ++db)
#pragma unroll
                                for (int r = 0; r < 16; ++r) o[0][db][r] *= alpha;
                            m_run = m_new;
                        }
                        float ls = fa::kSumInit;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            s[r] = fast_exp2(s[r] - m_run);
                            ls += s[r];
                        }
                        l_run += ls;  // this lane half's partial; the halves are summed after the sweep
                        T::template rchain<1>(o, vt, &s, c, hf, dh);
                    } else if constexpr (MODE == 1) {
                        const float m_new = fa::vmax(m_run, fa::tile_max(s));
                        float ls = fa::kSumInit;
#pragma unroll
                        for (int r = 0; r < 16; ++r) ls += fast_exp2(s[r] - m_new);
                        l_run = l_run * fast_exp2(m_run - m_new) + fa::halves_sum(ls);
                        m_run = m_new;
                    } else {
#pragma unroll
                        for (int r = 0; r < 16; ++r) s[r] = fast_exp2(s[r] - mlog);
                        // wave dh stores register group gs (keys 8*gs + 4h .. +3): DH = 4,
                        // gs = dh; DH = 8, gs = dh / 2 on the lane half h = dh % 2
                        const int gs = DH == 4 ? dh : dh >> 1;
                        if (qi < Sq && (DH == 4 || hf == (dh & 1))) {
                            const int k0 = t * BK + 8 * gs + 4 * hf;
                            floatx4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int g = 0; g < 4; ++g)
                                if (g == gs) v = floatx4{s[4 * g], s[4 * g + 1], s[4 * g + 2], s[4 * g + 3]};
                            if (pvec && k0 + 3 < Sk) {
                                *reinterpret_cast<floatx4*>(prow + k0) = v;
                            } else {
#pragma unroll
                                for (int j = 0; j < 4; ++j)
                                    if (k0 + j < Sk) prow[k0 + j] = v[j];
                            }
                        }
                        T::template rchain<1>(o, vt, &s, c, hf, dh);
                    }
                }
                __syncthreads();  // every wave is done with the stage and the exchange
                if (t + 1 < nstages) {
                    stg.store(lds, T::ROW, tid);
                    __syncthreads();
                }
            }
        };

        if constexpr (!PROBS) {
            sweep(std::integral_constant<int, 0>{}, 0.f, nullptr, false);
            l_run = fa::halves_sum(l_run);
        } else {
            float* const probs_bh = a.probs + (int64_t)bh * Sq * Sk;
            const bool pvec = (Sk & 3) == 0 && (reinterpret_cast<uintptr_t>(a.probs) & 15) == 0;
            // causal: the zeros above the diagonal need no data
            if (CAUSAL && qw0 < Sq && dh == 0)
                fa::zero_probs_tail(probs_bh, qw0, Sq, Sk, wtiles * BK, lane, pvec);
            sweep(std::integral_constant<int, 1>{}, 0.f, nullptr, false);
            const float mlog = m_run + __builtin_amdgcn_logf(fmaxf(l_run, 1e-20f));
            sweep(std::integral_constant<int, 2>{}, mlog, probs_bh + (int64_t)qi * Sk, pvec);
            l_run = 1.0f;  // P carries 1 / l already
        }

        if (!PROBS && a.lse && dh == 0 && hf == 0 && qi < Sq)
            a.lse[(int64_t)bh * Sq + qi] = (m_run + log2f(l_run)) * kLn2;
        if (qi < Sq) {
            const float linv = PROBS ? 1.0f : __builtin_amdgcn_rcpf(fmaxf(l_run, 1e-20f));
            float* orow = a.o + b * a.o_bs + h * a.o_hs + (int64_t)qi * a.o_ts;
#pragma unroll
            for (int db = 0; db < T::NDBW; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d0 = dh * T::DW + db * 32 + 8 * g + 4 * hf;
                    if (d0 < D)
                        *reinterpret_cast<floatx4*>(orow + d0) =
                            floatx4{o[0][db][4 * g] * linv, o[0][db][4 * g + 1] * linv, o[0][db][4 * g + 2] * linv,
                                    o[0][db][4 * g + 3] * linv};
                }
        }
    }
};

template <int DP, int DH, int NQB, bool CAUSAL, bool PROBS>
__global__ __launch_bounds__(NQB* DH * 64) void fa_wide_kernel(AttnArgs a) {
    using K = WideFwd<DP, DH, NQB, CAUSAL, PROBS>;
    __shared__ __attribute__((aligned(16))) float lds[K::LDS_FLOATS];
    K::run(a, lds);
}

// Eight waves per workgroup: padded D = 256 two query sub-blocks of four
// waves, D = 512 one of eight.
template <int DP, int DH, int NQB, bool CAUSAL, bool PROBS>
hipError_t launch_wide_one(const AttnArgs& a, hipStream_t s) {
    AttnArgs args = a;
    args.n_qblk = (a.Sq + NQB * QW - 1) / (NQB * QW);
    const int64_t grid = (int64_t)args.n_qblk * a.B * a.H;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((fa_wide_kernel<DP, DH, NQB, CAUSAL, PROBS>), dim3((unsigned)grid), dim3(NQB * DH * 64), 0, s,
                       args);
    return hipGetLastError();
}

template <bool CAUSAL, bool PROBS>
hipError_t launch_wide(const AttnArgs& a, hipStream_t s) {
    return a.D <= 256 ? launch_wide_one<256, 4, 2, CAUSAL, PROBS>(a, s) : launch_wide_one<512, 8, 1, CAUSAL, PROBS>(a, s);
}

}  // namespace

bool fa_wide_supported(int D) { return D > 128 && D <= 512 && D % 4 == 0; }

hipError_t launch_fa_wide(const AttnArgs& a, bool causal, hipStream_t stream) {
    if (!fa_wide_supported(a.D)) return hipErrorInvalidValue;
    const bool probs = a.probs != nullptr;
    if (causal) return probs ? launch_wide<true, true>(a, stream) : launch_wide<true, false>(a, stream);
    return probs ? launch_wide<false, true>(a, stream) : launch_wide<false, false>(a, stream);
}

}  // namespace hipgpt
