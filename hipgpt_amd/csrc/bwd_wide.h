// bwd_wide.h -- LDS-tiled MFMA kernels of the attention backward on the
// forward's probabilities (HipGPT src/hip_kernels.cpp:1159-1272) for the head
// dims the per-wave kernels of bwd_tiled.h do not take: padded head dims 128
// and 256 (whose per-wave accumulators and dO / V rows would not fit one
// wave's registers) and head dims below 64 that are not 32 or 64, any D with
// D % 4 == 0 and 16-byte aligned rows.
//
// Same math and the same two kernels as bwd_tiled.h (query-stationary dQ and
// row dots Dq through A = (P o dP) K and Bm = P K; key-stationary dK, dV with
// P and dS kept in registers), with the head dim split over DH waves: the DH
// waves of a sub-block share its 32 queries (resp. keys) and each holds and
// produces DW = DP / DH of the head dims.  The score-shaped products (dP) need
// every head dim, so each wave forms its partial dP over its own dims, the DH
// partials go through LDS, and every wave of the sub-block adds them in the
// same order (bit-identical totals).  Everything per wave then has the size of
// a DW-dim problem: DP = 128 runs DH = 2, DP = 256 DH = 4 (64 dims per wave).
// Operand tiles are row-major in LDS (pitch DP + 4: conflict-free
// ds_read_b128 along the head dim for dP); the products that contract over
// the tile's rows read them as single floats (one row per MFMA step, 32
// consecutive head dims across the lanes), so no transposed copies are
// staged.  Dims D..DP-1 are zero in every operand.  Causal (probs zero above
// the diagonal) skips tiles the same way bwd_tiled.h does.
// Recompute mode (RECOMP; the probs-free pair): P is rebuilt per tile as
// exp2(S' - lse'), S' = (scale log2 e) q.k formed like dP (a partial per
// wave, summed through LDS; K, resp. Q, is already a row-major stage tile),
// and Dq_i = dO_i . O_i.  The query-stationary kernel forms Dq from the rows
// of dO and O, stores it to the B*H*S workspace for the key-stationary
// kernel, and accumulates dQ = scale dS K directly.
#pragma once

#include "common.h"
#include "fa_common.h"
#include "kernels.h"
#include "rowtiles.h"

namespace hipgpt {
namespace bwd {

using fa::acc_key;
using fa::BK;
using fa::halves_sum;

// ----------------------------------------------------------------- dQ, Dq
// Workgroup: NQB query sub-blocks x DH dim slices; NBUF stage buffers (2:
// the next stage goes to the other buffer during the MFMAs; 1: it waits in
// registers and is stored after a barrier).
template <int DP, int NQB, int DH, int NBUF, bool CAUSAL, bool RECOMP>
struct WideQ {
    using T = RowTiles<DP, DH>;
    static constexpr int NW = NQB * DH;
    static constexpr int NT = NW * 64;
    static constexpr int STAGE = 2 * T::ROW;  // V, K (row-major)
    static constexpr int NACC = RECOMP ? 1 : 2;  // accumulators: A (, Bm)
    static constexpr int XCH = DH > 1 ? NW * 16 * 64 * (RECOMP ? 2 : 1) : 0;  // partial dP (, S') tiles
    static constexpr int LDS_FLOATS = NBUF * STAGE + XCH;

    __device__ __forceinline__ static void run(const BwdArgs& a, float* lds, int nqb, int bh, int rank) {
        const int tid = threadIdx.x, lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int c = lane & 31, hf = lane >> 5;
        const int sb = wave / DH, dh = wave % DH;
        const int qb = CAUSAL ? nqb - 1 - rank : rank;
        const int b = bh / a.H, h = bh % a.H;
        const int S = a.S, D = a.D;
        const int q0 = qb * NQB * BK, qw0 = q0 + sb * BK, qi = qw0 + c;
        const int64_t base = (int64_t)b * a.bs + (int64_t)h * a.hs;
        const int kend = CAUSAL ? min(S, q0 + NQB * BK) : S;
        const int nstages = (kend + BK - 1) / BK;
        const int wtiles = qw0 < S ? (CAUSAL ? (min(S, qw0 + BK) + BK - 1) / BK : nstages) : 0;

        float go[T::DW / 2];  // B operand of dP^T = V dO^T: dO[qi][wave's dims]
        T::load_lane_row(go, a.go + base, qi, S, D, a.ts, dh, hf);
        // Recompute mode: Q (B operand of S'^T = K Q^T) in log2 units, the
        // row's lse in the same units, and Dq_i = dO_i . O_i over every head
        // dim (the same sum in each of the DH waves).
        float q2[RECOMP ? T::DW / 2 : 1];
        float lse2 = 0.f, dqv = 0.f;
        if constexpr (RECOMP) {
            T::load_lane_row(q2, a.q + base, qi, S, D, a.ts, dh, hf);
            const float qsc = a.scale * kLog2e;
#pragma unroll
            for (int s2 = 0; s2 < T::DW / 2; ++s2) q2[s2] *= qsc;
            float dsum = 0.f;
            if (qi < S) {
                const float* gp = a.go + base + (int64_t)qi * a.ts;
                const float* op = a.o + base + (int64_t)qi * a.ts;
                for (int d0 = hf * 4; d0 < D; d0 += 8) {
                    const floatx4 g4 = *reinterpret_cast<const floatx4*>(gp + d0);
                    const floatx4 o4 = *reinterpret_cast<const floatx4*>(op + d0);
#pragma unroll
                    for (int j = 0; j < 4; ++j) dsum = fmaf(g4[j], o4[j], dsum);
                }
                lse2 = a.lse[(int64_t)bh * S + qi] * kLog2e;
            }
            dqv = halves_sum(dsum);
        }
        RowLoader vl, kl;
        vl.init(a.v + base, a.ts, S, D);
        kl.init(a.k + base, a.ts, S, D);
        RowStage<DP, NT, 2> stg;
        floatx4* const xch = reinterpret_cast<floatx4*>(lds + NBUF * STAGE);

        floatx16 acc[NACC][T::NDBW];  // A^T (recompute: dS K), Bm^T: [d][query]
#pragma unroll
        for (int n = 0; n < NACC; ++n)
#pragma unroll
            for (int db = 0; db < T::NDBW; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[n][db][r] = 0.f;
        float ld = 0.f;
        const float* prow = RECOMP ? nullptr : a.probs + ((int64_t)bh * S + qi) * S;
        const bool pvec = (S & 3) == 0;
        // P of key tile t in accumulator order (register 4g + j <-> key t*32 + 8g + 4h + j)
        auto load_p = [&](floatx4 (&pv)[4], int t) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int k0 = t * BK + 8 * g + 4 * hf;
                if (pvec && qi < S && k0 + 3 < S) {
                    pv[g] = *reinterpret_cast<const floatx4*>(prow + k0);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) pv[g][j] = (qi < S && k0 + j < S) ? prow[k0 + j] : 0.f;
                }
            }
        };
        floatx4 pnext[4];
        if (!RECOMP && wtiles > 0) load_p(pnext, 0);

        if (nstages > 0) {
            stg.load(vl, kl, 0, D, tid);
            stg.store(lds, T::ROW, tid);
        }
        __syncthreads();
        for (int st = 0; st < nstages; ++st) {
            const float* cur = lds + (NBUF == 2 ? (st & 1) * STAGE : 0);
            if (st + 1 < nstages) stg.load(vl, kl, (st + 1) * BK, D, tid);
            const bool act = st < wtiles;  // wave-uniform
            floatx16 dp;
#pragma unroll
            for (int r = 0; r < 16; ++r) dp[r] = 0.f;
            floatx16 sc;  // recompute mode: S'^T, register r <-> key acc_key(r, h)
#pragma unroll
            for (int r = 0; r < 16; ++r) sc[r] = 0.f;
            if (act) {
                T::dchain(dp, cur, go, c, hf, dh);  // (partial) dP^T, register r <-> key acc_key(r, h)
                if (RECOMP) T::dchain(sc, cur + T::ROW, q2, c, hf, dh);
            }
            if constexpr (DH > 1) {
                if (act) {
                    T::publish(dp, xch, wave, lane);
                    if (RECOMP) T::publish(sc, xch + NW * 256, wave, lane);
                }
                __syncthreads();
                if (act) {
                    dp = T::total(dp, xch, sb, dh, lane);
                    if (RECOMP) sc = T::total(sc, xch + NW * 256, sb, dh, lane);
                }
            }
            if constexpr (RECOMP) {
                if (act) {
                    const int kb0 = st * BK;
                    const bool edge = kb0 + BK > S || (CAUSAL && kb0 + BK - 1 > qw0);
                    floatx16 x;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = kb0 + acc_key(r, hf);
                        const float p = fast_exp2(sc[r] - lse2);
                        x[r] = (!edge || (key < S && (!CAUSAL || key <= qi))) ? p * (dp[r] - dqv) : 0.f;
                    }
                    T::template rchain<1>(acc, cur + T::ROW, &x, c, hf, dh);  // (dS K)^T += K^T dS^T
                }
            } else if (act) {
                floatx16 x[2];
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                    for (int j = 0; j < 4; ++j) x[1][4 * g + j] = pnext[g][j];
                if (st + 1 < wtiles) load_p(pnext, st + 1);
                float s = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    x[0][r] = x[1][r] * dp[r];
                    s += x[0][r];
                }
                ld += s;
                T::template rchain<2>(acc, cur + T::ROW, x, c, hf, dh);  // A^T += K^T (P o dP)^T, Bm^T += K^T P^T
            }
            if constexpr (NBUF == 2) {
                if (st + 1 < nstages) stg.store(lds + ((st + 1) & 1) * STAGE, T::ROW, tid);
                __syncthreads();
            } else {
                __syncthreads();
                if (st + 1 < nstages) {
                    stg.store(lds, T::ROW, tid);
                    __syncthreads();
                }
            }
        }

        const float dq = RECOMP ? dqv : halves_sum(ld);
        if (qi < S) {
            if (dh == 0 && hf == 0) a.dvec[(int64_t)bh * S + qi] = dq;
            float* out = a.dq + base + (int64_t)qi * a.ts;
#pragma unroll
            for (int db = 0; db < T::NDBW; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d0 = dh * T::DW + db * 32 + 8 * g + 4 * hf;
                    if (d0 < D) {
                        floatx4 v;
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            v[j] = RECOMP ? a.scale * acc[0][db][4 * g + j]
                                          : a.scale * fmaf(-dq, acc[NACC - 1][db][4 * g + j], acc[0][db][4 * g + j]);
                        *reinterpret_cast<floatx4*>(out + d0) = v;
                    }
                }
        }
    }
};

// ----------------------------------------------------------------- dK, dV
template <int DP, int NKB, int DH, int NBUF, bool CAUSAL, bool RECOMP>
struct WideKV {
    using T = RowTiles<DP, DH>;
    static constexpr int NW = NKB * DH;
    static constexpr int NT = NW * 64;
    static constexpr int DQ_OFF = 2 * T::ROW;
    static constexpr int LSE_OFF = DQ_OFF + BK;
    static constexpr int STAGE = 2 * T::ROW + BK + (RECOMP ? BK : 0);  // dO, Q (row-major), Dq (, lse')
    static constexpr int XCH = DH > 1 ? NW * 16 * 64 * (RECOMP ? 2 : 1) : 0;  // partial dP (, S') tiles
    static constexpr int LDS_FLOATS = NBUF * STAGE + XCH;
    static_assert(STAGE % 4 == 0, "16-byte aligned stage buffers");

    __device__ __forceinline__ static void run(const BwdArgs& a, float* lds, int bh, int rank) {
        const int tid = threadIdx.x, lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int c = lane & 31, hf = lane >> 5;
        const int sb = wave / DH, dh = wave % DH;
        const int kb = rank;  // causal: key block 0 sees the most query tiles and launches first
        const int b = bh / a.H, h = bh % a.H;
        const int S = a.S, D = a.D;
        const int k0 = kb * NKB * BK, kw0 = k0 + sb * BK, kj = kw0 + c;
        const int64_t base = (int64_t)b * a.bs + (int64_t)h * a.hs;
        const int nq = (S + BK - 1) / BK;
        const int it0 = CAUSAL ? k0 / BK : 0;
        const int wit0 = CAUSAL ? kw0 / BK : 0;
        const int nstages = nq - it0;

        float vr[T::DW / 2];  // B operand of dP = dO V^T: V[kj][wave's dims]
        T::load_lane_row(vr, a.v + base, kj, S, D, a.ts, dh, hf);
        // Recompute mode: K (B operand of S' = Q K^T) in log2 units
        float kr2[RECOMP ? T::DW / 2 : 1];
        if constexpr (RECOMP) {
            T::load_lane_row(kr2, a.k + base, kj, S, D, a.ts, dh, hf);
            const float qsc = a.scale * kLog2e;
#pragma unroll
            for (int s2 = 0; s2 < T::DW / 2; ++s2) kr2[s2] *= qsc;
        }
        RowLoader gl, ql;
        gl.init(a.go + base, a.ts, S, D);
        ql.init(a.q + base, a.ts, S, D);
        RowStage<DP, NT, 2> stg;
        float dqs = 0.f;
        float lses = 0.f;  // recompute mode: lse' of the staged row (+inf past the last row: P = 0)
        floatx4* const xch = reinterpret_cast<floatx4*>(lds + NBUF * STAGE);

        floatx16 acc[2][T::NDBW];  // dV^T, dK^T (unscaled): [d][key]
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int db = 0; db < T::NDBW; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[n][db][r] = 0.f;
        const float* pcol = RECOMP ? nullptr : a.probs + (int64_t)bh * S * S + kj;
        // P column of query tile it, register r <-> query it*32 + acc_key(r, h)
        auto load_p = [&](floatx16& pv, int it) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int qr = it * BK + acc_key(r, hf);
                pv[r] = (qr < S && kj < S) ? pcol[(int64_t)qr * S] : 0.f;
            }
        };
        auto load = [&](int st) {
            const int row0 = (it0 + st) * BK;
            stg.load(gl, ql, row0, D, tid);
            if (tid < BK) {
                dqs = row0 + tid < S ? a.dvec[(int64_t)bh * S + row0 + tid] : 0.f;
                if (RECOMP) lses = row0 + tid < S ? a.lse[(int64_t)bh * S + row0 + tid] * kLog2e : kInf;
            }
        };
        auto store = [&](float* dst) {
            stg.store(dst, T::ROW, tid);
            if (tid < BK) {
                dst[DQ_OFF + tid] = dqs;
                if (RECOMP) dst[LSE_OFF + tid] = lses;
            }
        };
        floatx16 pnext;
        if (!RECOMP && wit0 < nq) load_p(pnext, wit0);

        if (nstages > 0) {
            load(0);
            store(lds);
        }
        __syncthreads();
        for (int st = 0; st < nstages; ++st) {
            const float* cur = lds + (NBUF == 2 ? (st & 1) * STAGE : 0);
            if (st + 1 < nstages) load(st + 1);
            const int it = it0 + st;
            const bool act = it >= wit0;  // wave-uniform
            floatx16 dp;
#pragma unroll
            for (int r = 0; r < 16; ++r) dp[r] = 0.f;
            floatx16 sc;  // recompute mode: S', register r <-> query acc_key(r, h)
#pragma unroll
            for (int r = 0; r < 16; ++r) sc[r] = 0.f;
            if (act) {
                T::dchain(dp, cur, vr, c, hf, dh);  // (partial) dP, register r <-> query acc_key(r, h)
                if (RECOMP) T::dchain(sc, cur + T::ROW, kr2, c, hf, dh);
            }
            if constexpr (DH > 1) {
                if (act) {
                    T::publish(dp, xch, wave, lane);
                    if (RECOMP) T::publish(sc, xch + NW * 256, wave, lane);
                }
                __syncthreads();
                if (act) {
                    dp = T::total(dp, xch, sb, dh, lane);
                    if (RECOMP) sc = T::total(sc, xch + NW * 256, sb, dh, lane);
                }
            }
            if (act) {
                floatx16 x[2];  // P, dS
                if constexpr (RECOMP) {
                    // causal: some query of this tile precedes some key of the wave
                    const bool edge = CAUSAL && it * BK < kw0 + BK - 1;
                    const float* lt = cur + LSE_OFF;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const floatx4 l4 = *reinterpret_cast<const floatx4*>(lt + 8 * g + 4 * hf);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const float p = fast_exp2(sc[4 * g + j] - l4[j]);
                            x[0][4 * g + j] = (!edge || it * BK + 8 * g + 4 * hf + j >= kj) ? p : 0.f;
                        }
                    }
                } else {
                    x[0] = pnext;
                    if (it + 1 < nq) load_p(pnext, it + 1);
                }
                const float* dqt = cur + DQ_OFF;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const floatx4 dq = *reinterpret_cast<const floatx4*>(dqt + 8 * g + 4 * hf);
#pragma unroll
                    for (int j = 0; j < 4; ++j) x[1][4 * g + j] = x[0][4 * g + j] * (dp[4 * g + j] - dq[j]);
                }
                T::template rchain<1>(&acc[0], cur, &x[0], c, hf, dh);           // dV^T += dO^T P
                T::template rchain<1>(&acc[1], cur + T::ROW, &x[1], c, hf, dh);  // dK^T += Q^T dS
            }
            if constexpr (NBUF == 2) {
                if (st + 1 < nstages) store(lds + ((st + 1) & 1) * STAGE);
                __syncthreads();
            } else {
                __syncthreads();
                if (st + 1 < nstages) {
                    store(lds);
                    __syncthreads();
                }
            }
        }

        if (kj < S) {
            float* dvp = a.dv + base + (int64_t)kj * a.ts;
            float* dkp = a.dk + base + (int64_t)kj * a.ts;
#pragma unroll
            for (int db = 0; db < T::NDBW; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d0 = dh * T::DW + db * 32 + 8 * g + 4 * hf;
                    if (d0 < D) {
                        *reinterpret_cast<floatx4*>(dvp + d0) = floatx4{acc[0][db][4 * g], acc[0][db][4 * g + 1],
                                                                        acc[0][db][4 * g + 2], acc[0][db][4 * g + 3]};
                        *reinterpret_cast<floatx4*>(dkp + d0) =
                            floatx4{a.scale * acc[1][db][4 * g], a.scale * acc[1][db][4 * g + 1],
                                    a.scale * acc[1][db][4 * g + 2], a.scale * acc[1][db][4 * g + 3]};
                    }
                }
        }
    }
};

template <int DP, int NQB, int DH, int NBUF, bool CAUSAL, bool RECOMP>
__global__ __launch_bounds__(NQB* DH * 64) void bwd_wide_q_kernel(BwdArgs a, int nqb) {
    using K = WideQ<DP, NQB, DH, NBUF, CAUSAL, RECOMP>;
    __shared__ __attribute__((aligned(16))) float lds[K::LDS_FLOATS];
    const int BH = a.B * a.H;
    K::run(a, lds, nqb, blockIdx.x % BH, blockIdx.x / BH);
}

template <int DP, int NKB, int DH, int NBUF, bool CAUSAL, bool RECOMP>
__global__ __launch_bounds__(NKB* DH * 64) void bwd_wide_kv_kernel(BwdArgs a) {
    using K = WideKV<DP, NKB, DH, NBUF, CAUSAL, RECOMP>;
    __shared__ __attribute__((aligned(16))) float lds[K::LDS_FLOATS];
    const int BH = a.B * a.H;
    K::run(a, lds, blockIdx.x % BH, blockIdx.x / BH);
}

// Both kernels of one problem (the second reads the first's Dq).  Blocks
// b run (b, h) = b mod B*H at launch rank b / B*H: the heaviest causal blocks
// of every (b, h) first.
template <int DP, int NB, int DH, int NBUF, bool CAUSAL, bool RECOMP>
hipError_t launch_wide_mode(const BwdArgs& a, hipStream_t s) {
    const int BH = a.B * a.H;
    const int nb = (a.S + NB * BK - 1) / (NB * BK);
    const int64_t g = (int64_t)nb * BH;
    if (g <= 0 || g > 0x7fffffff) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((bwd_wide_q_kernel<DP, NB, DH, NBUF, CAUSAL, RECOMP>), dim3((unsigned)g), dim3(NB * DH * 64), 0,
                       s, a, nb);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_wide_kv_kernel<DP, NB, DH, NBUF, CAUSAL, RECOMP>), dim3((unsigned)g), dim3(NB * DH * 64),
                       0, s, a);
    return hipGetLastError();
}

// Stored probs, or (probs == nullptr) recompute mode from a.o and a.lse; both
// need the B*H*S workspace a.dvec.
template <int DP, int NB, int DH, int NBUF>
hipError_t launch_wide(const BwdArgs& a, hipStream_t s) {
    if (!a.probs)
        return a.causal ? launch_wide_mode<DP, NB, DH, NBUF, true, true>(a, s)
                        : launch_wide_mode<DP, NB, DH, NBUF, false, true>(a, s);
    return a.causal ? launch_wide_mode<DP, NB, DH, NBUF, true, false>(a, s)
                    : launch_wide_mode<DP, NB, DH, NBUF, false, false>(a, s);
}

}  // namespace bwd
}  // namespace hipgpt
