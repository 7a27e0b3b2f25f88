// bwd_tiled.h -- LDS-tiled MFMA kernels of the attention backward on the
// forward's probabilities (HipGPT src/hip_kernels.cpp:1159-1272), for head
// dims 32 and 64 with 16-byte aligned rows.
//
// Math per (b, h), scale c = 1/sqrt(D):
//   dP = dO V^T,  Dq_i = sum_j P_ij dP_ij,  dS = P o (dP - Dq),
//   dQ = c dS K,  dK = c dS^T Q,  dV = P^T dO.
// Two kernels, every gradient element written once (no atomics, no memset):
//   * bwd_q_kernel (query-stationary): wave (qs, ks) owns 32 queries and every
//     NKS-th key tile.  One pass over the keys accumulates
//       A = (P o dP) K,  Bm = P K,  Dq = rowsum(P o dP),
//     and dQ = c (A - Dq Bm), so P and V are read once; the key splits are
//     summed through LDS.  Dq goes to the workspace for the second kernel.
//   * bwd_kv_kernel (key-stationary): wave (ks, qs) owns 32 keys (V in
//     registers) and every NQS-th query tile; dP = dO V^T lands with one key
//     per lane and the queries in the accumulator's register order, which is
//     the B-operand layout of dV^T += dO^T P and dK^T += Q^T dS, so P and dS
//     never leave registers; the query splits are summed through LDS.
// Operand tiles go global -> registers -> LDS, double buffered, one barrier
// per stage (one key tile, resp. NQS query tiles), with the next stage's
// loads in flight during the MFMAs.  LDS tiles are row-major (pitch DP+4:
// conflict-free ds_read_b128 along the head dim) or transposed (pitch 36:
// ds_read_b128 along the 32 rows).  P is read straight from global memory in
// the layout each kernel needs: rows of 16 bytes (query-stationary) or
// 128-byte row segments per half-wave (key-stationary).
// Causal (probs zero above the diagonal) skips key tiles past a query
// tile's diagonal (query-stationary) and query tiles before a key tile's
// diagonal (key-stationary).
// Recompute mode (RECOMP; FlashAttention-2's backward): no probs buffer.  The
// forward's O and row log-sum-exp give Dq_i = dO_i . O_i up front (each kernel
// forms it from the dO rows it loads; the query-stationary one then forms
// dQ = c dS K directly) and P is rebuilt per tile as exp2(S' - lse'),
// S' = (c log2 e) q.k from the operand tiles already in LDS plus a row-major K
// (resp. Q) tile, with the causal mask applied on the diagonal tiles.  As
// neither kernel then reads the other's output, bwd_pair_kernel runs both
// kinds of workgroup in one launch.
#pragma once

#include <type_traits>

#include "common.h"
#include "fa_common.h"
#include "kernels.h"

namespace hipgpt {
namespace bwd {

using fa::acc_key;
using fa::BK;
using fa::halves_sum;

constexpr int TP = BK + 4;  // pitch of a transposed tile (rows are head dims)

template <int DP>
struct Tiles {
    static constexpr int RP = DP + 4;           // pitch of a row-major tile
    static constexpr int ROW = BK * RP;         // floats of a row-major tile
    static constexpr int TR = DP * TP;          // floats of a transposed tile
    static constexpr int CPR = DP / 4;          // 16-byte chunks per row
    static constexpr int CPT = BK * CPR;        // chunks per tile

    __device__ __forceinline__ static void store_row(float* t, int r, int cc, const floatx4& v) {
        *reinterpret_cast<floatx4*>(t + r * RP + cc * 4) = v;
    }
    __device__ __forceinline__ static void store_tr(float* t, int r, int cc, const floatx4& v) {
#pragma unroll
        for (int j = 0; j < 4; ++j) t[(cc * 4 + j) * TP + r] = v[j];
    }
    // Chain over the head dim: D[m = row c of `rt`][n = c] += sum_d rt[c][d] b[d],
    // lane (c, h) taking d = h*DP/2 + s (b holds the lane's DP/2 values).
    __device__ __forceinline__ static void dchain(floatx16& acc, const float* rt, const float* b, int c, int hf) {
        const float* rr = rt + c * RP + hf * (DP / 2);
#pragma unroll
        for (int j = 0; j < DP / 8; ++j) {
            const floatx4 kv = *reinterpret_cast<const floatx4*>(rr + 4 * j);
#pragma unroll
            for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[u], b[4 * j + u], acc, 0, 0, 0);
        }
    }
    // Chain over the 32 tile rows: acc[n][db][m = d][n = c] += sum_k tt[d][k] x[n][k][c]
    // for N right-hand operands sharing the A tile, x in accumulator register
    // order (register t <-> row acc_key(t, h)).
    template <int N>
    __device__ __forceinline__ static void rchain(floatx16 (*acc)[DP / 32], const float* tt, const floatx16* x, int c,
                                                  int hf) {
#pragma unroll
        for (int db = 0; db < DP / 32; ++db) {
            const float* p = tt + (db * 32 + c) * TP + 4 * hf;
            floatx4 blk[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) blk[g] = *reinterpret_cast<const floatx4*>(p + 8 * g);
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int n = 0; n < N; ++n)
                        acc[n][db] = __builtin_amdgcn_mfma_f32_32x32x2f32(blk[g][u], x[n][4 * g + u], acc[n][db], 0, 0, 0);
        }
    }
};

// Wave role from its SIMD rank sr and the workgroup's launch rank.  The
// launch ranks of one (b, h) are dealt to the same CUs in turn, so a CU holds
// one workgroup of each rank.  Rotating the roles by the rank spreads causal
// work when there are as many ranks as roles; with two ranks (the c1 / c2
// shapes: 4 roles of 5..8 and 1..4 tiles, resp. 8..5 and 4..1) the second rank
// takes the roles in reverse SIMD order, so every SIMD carries 9 tiles instead
// of 7..11.
__device__ __forceinline__ int role_of(int sr, int rank, int nranks, int nw, bool causal) {
    if (causal && nranks == 2) return rank ? nw - 1 - sr : sr;
    return (sr + rank) % nw;
}

// ----------------------------------------------------------------- dQ, Dq
template <int DP, int NQS, int NKS, bool CAUSAL, bool RECOMP>
struct BwdQ {
    using T = Tiles<DP>;
    static constexpr int NW = NQS * NKS;
    static constexpr int NT = NW * 64;
    static constexpr int NDB = DP / 32;
    static constexpr int NACC = RECOMP ? 1 : 2;  // accumulators: A (, Bm)
    // stage: NKS key tiles, each V row-major + K transposed (+ K row-major,
    // the A operand of S^T = K Q^T, when P is recomputed)
    static constexpr int KT = T::ROW + T::TR + (RECOMP ? T::ROW : 0);
    static constexpr int STAGE = NKS * KT;
    static constexpr int PER = (2 * NKS * T::CPT + NT - 1) / NT;  // chunks per thread per stage
    static constexpr int MERGE = NKS > 1 ? NW * 64 * (2 * 16 * NDB + 1) : 0;
    static constexpr int LDS_FLOATS = 2 * STAGE > MERGE ? 2 * STAGE : MERGE;

    // Workgroup `rank` of the nqb query blocks of problem bh.
    __device__ __forceinline__ static void run(const BwdArgs& a, float* lds, int* simd_slots, int nqb, int bh, int rank) {
        const int tid = threadIdx.x, lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int c = lane & 31, hf = lane >> 5;
        const int qb = CAUSAL ? nqb - 1 - rank : rank;
        const int role = role_of(fa::simd_rank<NW>(simd_slots, wave, lane), rank, nqb, NW, CAUSAL);
        const int qs = role / NKS, ks = role % NKS;
        const int b = bh / a.H, h = bh % a.H;
        const int S = a.S;
        const int q0 = qb * NQS * BK, qw0 = q0 + qs * BK, qi = qw0 + c;
        const int64_t base = (int64_t)b * a.bs + (int64_t)h * a.hs;
        const int kend = CAUSAL ? min(S, q0 + NQS * BK) : S;
        const int ntiles = (kend + BK - 1) / BK;
        const int wtiles = qw0 < S ? (CAUSAL ? (min(S, qw0 + BK) + BK - 1) / BK : ntiles) : 0;
        const int nstages = (ntiles + NKS - 1) / NKS;

        // dO (B operand of dP^T = V dO^T): lane (c, h) holds dO[qi][h*DP/2 + s]
        float go[DP / 2];
        {
            const float* g = a.go + base + (int64_t)qi * a.ts + hf * (DP / 2);
#pragma unroll
            for (int s = 0; s < DP / 2; s += 4) {
                const floatx4 t = qi < S ? *reinterpret_cast<const floatx4*>(g + s) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) go[s + j] = t[j];
            }
        }
        // Recompute mode: Q (B operand of S^T = K Q^T) pre-scaled to log2
        // units, the row's log-sum-exp in the same units, and the row dot
        // Dq_i = dO_i . O_i.
        float q2[RECOMP ? DP / 2 : 1];
        float lse2 = 0.f, dqv = 0.f;
        if constexpr (RECOMP) {
            const float qsc = a.scale * kLog2e;
            const float* qp = a.q + base + (int64_t)qi * a.ts + hf * (DP / 2);
            const float* op = a.o + base + (int64_t)qi * a.ts + hf * (DP / 2);
            float dsum = 0.f;
#pragma unroll
            for (int s = 0; s < DP / 2; s += 4) {
                const floatx4 qv = qi < S ? *reinterpret_cast<const floatx4*>(qp + s) : floatx4{0.f, 0.f, 0.f, 0.f};
                const floatx4 ov = qi < S ? *reinterpret_cast<const floatx4*>(op + s) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    q2[s + j] = qv[j] * qsc;
                    dsum = fmaf(go[s + j], ov[j], dsum);
                }
            }
            dqv = halves_sum(dsum);
            if (qi < S) lse2 = a.lse[(int64_t)bh * S + qi] * kLog2e;
        }
        RowLoader kl, vl;
        kl.init(a.k + base, a.ts, S, a.D);
        vl.init(a.v + base, a.ts, S, a.D);
        floatx4 stg[PER];
        static_assert((NKS * T::CPT) % 64 == 0, "a wave's chunks are all K or all V");
        auto load = [&](int st) {
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = tid + i * NT;
                if ((2 * NKS * T::CPT) % NT != 0 && f >= 2 * NKS * T::CPT) break;
                const int isk = f >= NKS * T::CPT;
                const int g = isk ? f - NKS * T::CPT : f;
                const int row = st * NKS * BK + g / T::CPR;
                // K or V is wave-uniform (NKS * CPT is a multiple of 64): a scalar
                // branch instead of a per-lane select of two buffer resources
                if (__builtin_amdgcn_readfirstlane(isk))
                    stg[i] = kl.load(row, g % T::CPR);
                else
                    stg[i] = vl.load(row, g % T::CPR);
            }
        };
        auto store = [&](float* dst) {
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = tid + i * NT;
                if ((2 * NKS * T::CPT) % NT != 0 && f >= 2 * NKS * T::CPT) break;
                const int isk = f >= NKS * T::CPT;
                const int g = isk ? f - NKS * T::CPT : f;
                const int kt = g / T::CPT, r = (g % T::CPT) / T::CPR, cc = g % T::CPR;
                float* tile = dst + kt * KT;
                if (isk) {
                    T::store_tr(tile + T::ROW, r, cc, stg[i]);
                    if (RECOMP) T::store_row(tile + T::ROW + T::TR, r, cc, stg[i]);
                } else {
                    T::store_row(tile, r, cc, stg[i]);
                }
            }
        };

        floatx16 acc[NACC][NDB];  // [0] = A^T (recompute: dS K, unscaled), [1] = Bm^T, both [d][query]
#pragma unroll
        for (int n = 0; n < NACC; ++n)
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[n][db][r] = 0.f;
        float ld = 0.f;
        const float* prow = RECOMP ? nullptr : a.probs + ((int64_t)bh * S + qi) * S;
        const bool pvec = (S & 3) == 0;

        // P of key tile t in accumulator order: piece g holds keys
        // t*32 + 8g + 4h .. +3 (register 4g + j <-> key t*32 + acc_key(4g + j, h)).
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
        // The next tile's P is requested while this tile's MFMAs run.
        floatx4 pnext[4];
        if (!RECOMP && ks < wtiles) load_p(pnext, ks);

        auto compute = [&](int st, const float* cur) {
            const int t = st * NKS + ks;
            if (t >= wtiles) return;
            const float* tile = cur + ks * KT;
            floatx16 x[2];
            if constexpr (RECOMP) {
                floatx16 sc;
#pragma unroll
                for (int r = 0; r < 16; ++r) sc[r] = 0.f;
                T::dchain(sc, tile + T::ROW + T::TR, q2, c, hf);  // S'^T, register r <-> key acc_key(r, h)
                const int kb0 = t * BK;
                const bool edge = kb0 + BK > S || (CAUSAL && kb0 + BK - 1 > qw0);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kb0 + acc_key(r, hf);
                    const float p = fast_exp2(sc[r] - lse2);
                    x[1][r] = (!edge || (key < S && (!CAUSAL || key <= qi))) ? p : 0.f;
                }
            } else {
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                    for (int j = 0; j < 4; ++j) x[1][4 * g + j] = pnext[g][j];
                if (t + NKS < wtiles) load_p(pnext, t + NKS);
            }
            floatx16 dp;
#pragma unroll
            for (int r = 0; r < 16; ++r) dp[r] = 0.f;
            T::dchain(dp, tile, go, c, hf);  // dP^T, register r <-> key acc_key(r, h)
            if constexpr (RECOMP) {
#pragma unroll
                for (int r = 0; r < 16; ++r) x[0][r] = x[1][r] * (dp[r] - dqv);
                T::template rchain<1>(acc, tile + T::ROW, x, c, hf);  // (dS K)^T += K^T dS^T
            } else {
                float s = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    x[0][r] = x[1][r] * dp[r];
                    s += x[0][r];
                }
                ld += s;
                T::template rchain<2>(acc, tile + T::ROW, x, c, hf);  // A^T += K^T (P o dP)^T, Bm^T += K^T P^T
            }
        };

        if (nstages > 0) {
            load(0);
            store(lds);
        }
        __syncthreads();
        for (int st = 0; st < nstages; ++st) {
            if (st + 1 < nstages) load(st + 1);
            compute(st, lds + (st & 1) * STAGE);
            if (st + 1 < nstages) store(lds + ((st + 1) & 1) * STAGE);
            __syncthreads();
        }

        // sum the key splits (wave ks == 0 keeps the sub-block)
        if (NKS > 1) {
            float* const mo = lds;  // [NW][2*16*NDB + 1][64]
            constexpr int W = 2 * 16 * NDB + 1;
            if (ks != 0) {
#pragma unroll
                for (int n = 0; n < NACC; ++n)
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
#pragma unroll
                        for (int r = 0; r < 16; ++r) mo[(role * W + (n * NDB + db) * 16 + r) * 64 + lane] = acc[n][db][r];
                mo[(role * W + W - 1) * 64 + lane] = ld;
            }
            __syncthreads();
            if (ks == 0) {
#pragma unroll
                for (int j = 1; j < NKS; ++j) {
#pragma unroll
                    for (int n = 0; n < NACC; ++n)
#pragma unroll
                        for (int db = 0; db < NDB; ++db)
#pragma unroll
                            for (int r = 0; r < 16; ++r)
                                acc[n][db][r] += mo[((role + j) * W + (n * NDB + db) * 16 + r) * 64 + lane];
                    ld += mo[((role + j) * W + W - 1) * 64 + lane];
                }
            }
        }
        if (ks == 0 && qi < S) {
            const float dq = RECOMP ? dqv : halves_sum(ld);
            if (!RECOMP && hf == 0) a.dvec[(int64_t)bh * S + qi] = dq;
            float* out = a.dq + base + (int64_t)qi * a.ts;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    floatx4 v;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        v[j] = RECOMP ? a.scale * acc[0][db][4 * g + j]
                                      : a.scale * fmaf(-dq, acc[NACC - 1][db][4 * g + j], acc[0][db][4 * g + j]);
                    *reinterpret_cast<floatx4*>(out + db * 32 + 8 * g + 4 * hf) = v;
                }
        }
    }
};

// ----------------------------------------------------------------- dK, dV
template <int DP, int NKB, int NQS, bool CAUSAL, bool RECOMP>
struct BwdKV {
    using T = Tiles<DP>;
    static constexpr int NW = NKB * NQS;
    static constexpr int NT = NW * 64;
    static constexpr int NDB = DP / 32;
    // stage: NQS query tiles, each dO row-major + dO transposed + Q transposed
    // + Dq (+ lse' + Q row-major, the A operand of S' = Q K^T, when P is
    // recomputed)
    static constexpr int DQ_OFF = T::ROW + 2 * T::TR;
    static constexpr int LSE_OFF = DQ_OFF + BK;
    static constexpr int QROW_OFF = LSE_OFF + BK;
    static constexpr int QT = DQ_OFF + BK + (RECOMP ? BK + T::ROW : 0);
    static constexpr int STAGE = NQS * QT;
    static constexpr int PER = (2 * NQS * T::CPT + NT - 1) / NT;
    static constexpr int MERGE = NQS > 1 ? NW * 64 * (2 * 16 * NDB) : 0;
    static constexpr int LDS_FLOATS = 2 * STAGE > MERGE ? 2 * STAGE : MERGE;
    // Recompute mode forms Dq from the staged dO chunks: chunks i < NG of a
    // thread are dO, and a row's CPR chunks sit in consecutive lanes.
    static constexpr int NG = NQS * T::CPT / NT;
    static_assert(!RECOMP || (NQS * T::CPT) % NT == 0, "dO chunks must fill whole passes");

    // Workgroup `rank` (the key block) of the nkb key blocks of problem bh.
    __device__ __forceinline__ static void run(const BwdArgs& a, float* lds, int* simd_slots, int nkb, int bh, int rank) {
        const int tid = threadIdx.x, lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int c = lane & 31, hf = lane >> 5;
        const int kb = rank;  // key block; causal: block 0 sees the most query tiles and launches first
        const int role = role_of(fa::simd_rank<NW>(simd_slots, wave, lane), rank, nkb, NW, CAUSAL);
        const int ksub = role / NQS, qsp = role % NQS;
        const int b = bh / a.H, h = bh % a.H;
        const int S = a.S;
        const int k0 = kb * NKB * BK, kw0 = k0 + ksub * BK, kj = kw0 + c;
        const int64_t base = (int64_t)b * a.bs + (int64_t)h * a.hs;
        const int nq = (S + BK - 1) / BK;
        // query tiles [it0, nq): causal starts at the workgroup's first key tile
        const int it0 = CAUSAL ? k0 / BK : 0;
        const int wit0 = CAUSAL ? kw0 / BK : 0;  // this wave's first useful query tile
        const int nstages = (nq - it0 + NQS - 1) / NQS;

        // V (B operand of dP = dO V^T): lane (c, h) holds V[kj][h*DP/2 + s]
        float vr[DP / 2];
        {
            const float* vp = a.v + base + (int64_t)kj * a.ts + hf * (DP / 2);
#pragma unroll
            for (int s = 0; s < DP / 2; s += 4) {
                const floatx4 t = kj < S ? *reinterpret_cast<const floatx4*>(vp + s) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) vr[s + j] = t[j];
            }
        }
        // Recompute mode: K (B operand of S' = Q K^T) pre-scaled to log2 units
        float kr2[RECOMP ? DP / 2 : 1];
        if constexpr (RECOMP) {
            const float qsc = a.scale * kLog2e;
            const float* kp = a.k + base + (int64_t)kj * a.ts + hf * (DP / 2);
#pragma unroll
            for (int s = 0; s < DP / 2; s += 4) {
                const floatx4 t = kj < S ? *reinterpret_cast<const floatx4*>(kp + s) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) kr2[s + j] = t[j] * qsc;
            }
        }
        RowLoader gl, ql, ol;
        gl.init(a.go + base, a.ts, S, a.D);
        ql.init(a.q + base, a.ts, S, a.D);
        if (RECOMP) ol.init(a.o + base, a.ts, S, a.D);
        floatx4 stg[PER];
        floatx4 ostg[RECOMP ? NG : 1];  // O chunks matching the dO chunks (recompute mode)
        float dqs = 0.f;   // Dq value this thread stages (stored-probs mode)
        float lses = 0.f;  // lse' value this thread stages (+inf past the last row: P = 0)
        static_assert((NQS * T::CPT) % 64 == 0, "a wave's chunks are all Q or all dO");
        auto load = [&](int st) {
            const int qt0 = it0 + st * NQS;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = tid + i * NT;
                if ((2 * NQS * T::CPT) % NT != 0 && f >= 2 * NQS * T::CPT) break;
                const int isq = f >= NQS * T::CPT;
                const int g = isq ? f - NQS * T::CPT : f;
                const int row = qt0 * BK + g / T::CPR;
                if (__builtin_amdgcn_readfirstlane(isq))  // wave-uniform, as above
                    stg[i] = ql.load(row, g % T::CPR);
                else
                    stg[i] = gl.load(row, g % T::CPR);
                if constexpr (RECOMP) {
                    if (i < NG) ostg[i] = ol.load(row, g % T::CPR);
                }
            }
            if (tid < NQS * BK) {
                const int qrow = qt0 * BK + tid;
                if (RECOMP)
                    lses = qrow < S ? a.lse[(int64_t)bh * S + qrow] * kLog2e : kInf;
                else
                    dqs = qrow < S ? a.dvec[(int64_t)bh * S + qrow] : 0.f;
            }
        };
        auto store = [&](float* dst) {
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = tid + i * NT;
                if ((2 * NQS * T::CPT) % NT != 0 && f >= 2 * NQS * T::CPT) break;
                const int isq = f >= NQS * T::CPT;
                const int g = isq ? f - NQS * T::CPT : f;
                const int qt = g / T::CPT, r = (g % T::CPT) / T::CPR, cc = g % T::CPR;
                float* tile = dst + qt * QT;
                if (isq) {
                    T::store_tr(tile + T::ROW + T::TR, r, cc, stg[i]);
                    if (RECOMP) T::store_row(tile + QROW_OFF, r, cc, stg[i]);
                } else {
                    T::store_row(tile, r, cc, stg[i]);
                    T::store_tr(tile + T::ROW, r, cc, stg[i]);
                }
                if constexpr (RECOMP) {
                    // Dq of row r: the chunk dots summed over the row's CPR lanes
                    // (rows past S load as zero: Dq = 0)
                    if (i < NG) {
                        float d = stg[i][0] * ostg[i][0];
#pragma unroll
                        for (int j = 1; j < 4; ++j) d = fmaf(stg[i][j], ostg[i][j], d);
#pragma unroll
                        for (int m = 1; m < T::CPR; m <<= 1) d += __shfl_xor(d, m);
                        if (cc == 0) tile[DQ_OFF + r] = d;
                    }
                }
            }
            if (tid < NQS * BK) {
                if (RECOMP)
                    dst[(tid / BK) * QT + LSE_OFF + tid % BK] = lses;
                else
                    dst[(tid / BK) * QT + DQ_OFF + tid % BK] = dqs;
            }
        };

        floatx16 acc[2][NDB];  // [0] = dV^T, [1] = dK^T (unscaled), both [d][key]
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int db = 0; db < NDB; ++db)
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
        // The wave's tiles are it = it0 + st*NQS + qsp for st = 0, 1, ...;
        // the next one's P is requested while this one's MFMAs run.
        floatx16 pnext;
        if (!RECOMP) {
            int it = it0 + qsp;
            while (it < wit0) it += NQS;
            if (it < nq) load_p(pnext, it);
        }

        auto compute = [&](int st, const float* cur) {
            const int it = it0 + st * NQS + qsp;
            if (it >= nq || it < wit0) return;
            const float* tile = cur + qsp * QT;
            floatx16 x[2];  // [0] = P, [1] = dS, register r <-> query it*32 + acc_key(r, h)
            if constexpr (RECOMP) {
                floatx16 sc;
#pragma unroll
                for (int r = 0; r < 16; ++r) sc[r] = 0.f;
                T::dchain(sc, tile + QROW_OFF, kr2, c, hf);  // S', register r <-> query acc_key(r, h)
                const float* lt = tile + LSE_OFF;
                // causal: some query of this tile precedes some key of the wave
                const bool edge = CAUSAL && it * BK < kw0 + BK - 1;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const floatx4 l4 = *reinterpret_cast<const floatx4*>(lt + 8 * g + 4 * hf);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float p = fast_exp2(sc[4 * g + j] - l4[j]);
                        x[0][4 * g + j] = (!edge || it * BK + acc_key(4 * g + j, hf) >= kj) ? p : 0.f;
                    }
                }
            } else {
                x[0] = pnext;
                if (it + NQS < nq) load_p(pnext, it + NQS);
            }
            floatx16 dp;
#pragma unroll
            for (int r = 0; r < 16; ++r) dp[r] = 0.f;
            T::dchain(dp, tile, vr, c, hf);  // dP, register r <-> query acc_key(r, h)
            const float* dqt = tile + DQ_OFF;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const floatx4 dq = *reinterpret_cast<const floatx4*>(dqt + 8 * g + 4 * hf);
#pragma unroll
                for (int j = 0; j < 4; ++j) x[1][4 * g + j] = x[0][4 * g + j] * (dp[4 * g + j] - dq[j]);
            }
            // dV^T += dO^T P, dK^T += Q^T dS: two A tiles, one per product
            T::template rchain<1>(&acc[0], tile + T::ROW, &x[0], c, hf);
            T::template rchain<1>(&acc[1], tile + T::ROW + T::TR, &x[1], c, hf);
        };

        if (nstages > 0) {
            load(0);
            store(lds);
        }
        __syncthreads();
        for (int st = 0; st < nstages; ++st) {
            if (st + 1 < nstages) load(st + 1);
            compute(st, lds + (st & 1) * STAGE);
            if (st + 1 < nstages) store(lds + ((st + 1) & 1) * STAGE);
            __syncthreads();
        }

        if (NQS > 1) {
            float* const mo = lds;  // [NW][2*16*NDB][64]
            constexpr int W = 2 * 16 * NDB;
            if (qsp != 0) {
#pragma unroll
                for (int n = 0; n < 2; ++n)
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
#pragma unroll
                        for (int r = 0; r < 16; ++r) mo[(role * W + (n * NDB + db) * 16 + r) * 64 + lane] = acc[n][db][r];
            }
            __syncthreads();
            if (qsp == 0) {
#pragma unroll
                for (int j = 1; j < NQS; ++j)
#pragma unroll
                    for (int n = 0; n < 2; ++n)
#pragma unroll
                        for (int db = 0; db < NDB; ++db)
#pragma unroll
                            for (int r = 0; r < 16; ++r)
                                acc[n][db][r] += mo[((role + j) * W + (n * NDB + db) * 16 + r) * 64 + lane];
            }
        }
        if (qsp == 0 && kj < S) {
            float* dvp = a.dv + base + (int64_t)kj * a.ts;
            float* dkp = a.dk + base + (int64_t)kj * a.ts;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d0 = db * 32 + 8 * g + 4 * hf;
                    *reinterpret_cast<floatx4*>(dvp + d0) =
                        floatx4{acc[0][db][4 * g], acc[0][db][4 * g + 1], acc[0][db][4 * g + 2], acc[0][db][4 * g + 3]};
                    *reinterpret_cast<floatx4*>(dkp + d0) =
                        floatx4{a.scale * acc[1][db][4 * g], a.scale * acc[1][db][4 * g + 1],
                                a.scale * acc[1][db][4 * g + 2], a.scale * acc[1][db][4 * g + 3]};
                }
        }
    }
};

template <int DP, int NQS, int NKS, bool CAUSAL, bool RECOMP>
__global__ __launch_bounds__(NQS* NKS * 64) void bwd_q_kernel(BwdArgs a, int nqb) {
    using K = BwdQ<DP, NQS, NKS, CAUSAL, RECOMP>;
    __shared__ __attribute__((aligned(16))) float lds[K::LDS_FLOATS];
    __shared__ int simd_slots[NQS * NKS];
    const int BH = a.B * a.H;
    K::run(a, lds, simd_slots, nqb, blockIdx.x % BH, blockIdx.x / BH);
}

template <int DP, int NKB, int NQS, bool CAUSAL, bool RECOMP>
__global__ __launch_bounds__(NKB* NQS * 64) void bwd_kv_kernel(BwdArgs a, int nkb) {
    using K = BwdKV<DP, NKB, NQS, CAUSAL, RECOMP>;
    __shared__ __attribute__((aligned(16))) float lds[K::LDS_FLOATS];
    __shared__ int simd_slots[NKB * NQS];
    const int BH = a.B * a.H;
    K::run(a, lds, simd_slots, nkb, blockIdx.x % BH, blockIdx.x / BH);
}

// Recompute mode: the query- and key-stationary workgroups of the same shape
// in one grid, dealt in chunks of B*H workgroups as query rank 0, key rank 0,
// query rank 1, ... (the heaviest causal blocks of each kind first), so that
// both kinds share the CUs -- twice the waves in flight of either kernel
// alone -- and the pair costs one launch.
template <int DP, int NQS, int NKS, int NKB, int NQS2, bool CAUSAL>
__global__ __launch_bounds__(NQS* NKS * 64) void bwd_pair_kernel(BwdArgs a, int nr) {
    using KQ = BwdQ<DP, NQS, NKS, CAUSAL, true>;
    using KK = BwdKV<DP, NKB, NQS2, CAUSAL, true>;
    static_assert(NQS * NKS == NKB * NQS2 && NQS == NKB, "both kinds need the same workgroup and block counts");
    constexpr int LF = KQ::LDS_FLOATS > KK::LDS_FLOATS ? KQ::LDS_FLOATS : KK::LDS_FLOATS;
    __shared__ __attribute__((aligned(16))) float lds[LF];
    __shared__ int simd_slots[NQS * NKS];
    const int BH = a.B * a.H;
    const int chunk = blockIdx.x / BH, bh = blockIdx.x % BH;
    if (chunk & 1)
        KK::run(a, lds, simd_slots, nr, bh, chunk >> 1);
    else
        KQ::run(a, lds, simd_slots, nr, bh, chunk >> 1);
}

// Both kernels for one problem: stored probs, two launches (the second reads
// the first's Dq); recompute mode, one launch of the pair kernel.
template <int DP, int QNQS, int QNKS, int KNKB, int KNQS, bool CAUSAL, bool RECOMP>
hipError_t launch_tiled_mode(const BwdArgs& a, hipStream_t s) {
    const int BH = a.B * a.H;
    const int nqb = (a.S + QNQS * BK - 1) / (QNQS * BK);
    const int nkb = (a.S + KNKB * BK - 1) / (KNKB * BK);
    const int64_t g1 = (int64_t)nqb * BH, g2 = (int64_t)nkb * BH;
    if (g1 <= 0 || g1 + g2 > 0x7fffffff) return hipErrorInvalidConfiguration;
    if constexpr (RECOMP) {
        hipLaunchKernelGGL((bwd_pair_kernel<DP, QNQS, QNKS, KNKB, KNQS, CAUSAL>), dim3((unsigned)(g1 + g2)),
                           dim3(QNQS * QNKS * 64), 0, s, a, nqb);
        return hipGetLastError();
    } else {
        hipLaunchKernelGGL((bwd_q_kernel<DP, QNQS, QNKS, CAUSAL, false>), dim3((unsigned)g1), dim3(QNQS * QNKS * 64), 0,
                           s, a, nqb);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((bwd_kv_kernel<DP, KNKB, KNQS, CAUSAL, false>), dim3((unsigned)g2), dim3(KNKB * KNQS * 64),
                           0, s, a, nkb);
        return hipGetLastError();
    }
}

// Stored probs: 4 x 1 workgroups, or 4 x 2 -- each query-stationary
// workgroup's keys and each key-stationary workgroup's queries split over two
// more waves, so a workgroup takes about half as long at half as many resident
// slots (one 8-wave workgroup per CU instead of two 4-wave ones; the same
// 128-row blocks, so the same grid).  The split pays when the 4 x 1 grid
// would end on a partly filled round: without a causal mask, when
// ceil(G / S2) / 2 (+10% for the wider workgroup) is below ceil(G / S1);
// causally (longest blocks first), when the whole grid fits one 4 x 2 round.
// Cache-rotated, D = 64: the HipGPT drop-in at B8 H12 S1024 (G = 768) 868 ->
// 737 us, B8 H8 S512 non-causal (G = 256) 148 -> 135, causal 142 -> 131;
// kept 4 x 1: non-causal B2 H12 S2048 (G = 384: 856 against 940 us), D = 32
// B8 H8 S1024 (G = 512: 259 against 285), causal B8 H12 S1024 (G = 768: 410
// against 436).  The probs-free pair keeps 4 x 1 (449 against 482 us at B8
// H12 S1024 causal).
template <int DP>
hipError_t launch_tiled_probs(const BwdArgs& a, hipStream_t s) {
    static ResidentSlots c1[2], c2[2];
    const int ci = a.causal ? 1 : 0;
    const void* k1 = a.causal ? reinterpret_cast<const void*>(bwd_q_kernel<DP, 4, 1, true, false>)
                              : reinterpret_cast<const void*>(bwd_q_kernel<DP, 4, 1, false, false>);
    const void* k2 = a.causal ? reinterpret_cast<const void*>(bwd_q_kernel<DP, 4, 2, true, false>)
                              : reinterpret_cast<const void*>(bwd_q_kernel<DP, 4, 2, false, false>);
    const int64_t S1 = c1[ci].get(k1, 4 * 64, 0), S2 = c2[ci].get(k2, 8 * 64, 0);
    const int64_t G = (int64_t)((a.S + 4 * BK - 1) / (4 * BK)) * a.B * a.H;
    bool split = false;
    if (S1 > 0 && S2 > 0)
        split = a.causal ? G <= S2 : 11 * ((G + S2 - 1) / S2) < 20 * ((G + S1 - 1) / S1);
    if (split)
        return a.causal ? launch_tiled_mode<DP, 4, 2, 4, 2, true, false>(a, s)
                        : launch_tiled_mode<DP, 4, 2, 4, 2, false, false>(a, s);
    return a.causal ? launch_tiled_mode<DP, 4, 1, 4, 1, true, false>(a, s)
                    : launch_tiled_mode<DP, 4, 1, 4, 1, false, false>(a, s);
}

template <int DP, int QNQS, int QNKS, int KNKB, int KNQS>
hipError_t launch_tiled(const BwdArgs& a, hipStream_t s) {
    const bool recomp = a.probs == nullptr;
    if (a.causal)
        return recomp ? launch_tiled_mode<DP, QNQS, QNKS, KNKB, KNQS, true, true>(a, s)
                      : launch_tiled_mode<DP, QNQS, QNKS, KNKB, KNQS, true, false>(a, s);
    return recomp ? launch_tiled_mode<DP, QNQS, QNKS, KNKB, KNQS, false, true>(a, s)
                  : launch_tiled_mode<DP, QNQS, QNKS, KNKB, KNQS, false, false>(a, s);
}

}  // namespace bwd
}  // namespace hipgpt
