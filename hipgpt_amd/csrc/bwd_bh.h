// bwd_bh.h -- attention backward with one workgroup per (b, h), for head
// dim 32 and S <= 256: the shape of HipGPT's default model
// (src/train_gpt.cpp:175-180), whose backward is src/hip_kernels.cpp:1159-1272.
// Two kernels: bwd_bh_kernel rebuilds P from the forward's O and row lse;
// bwd_bh_probs_kernel (below) reads the stored probs, the reference's
// contract.
//
// One (b, h) problem fits one CU: Q and dO rows, the row log-sum-exp and
// Dq = dO . O stay in LDS for the whole launch, and each of the 8 waves keeps
// its 32 keys (K, V) in registers.  The wave owning key tile j walks the
// query tiles (causal: from its diagonal on) and computes per 32x32 tile
//   S' = (c log2 e) Q K^T,  P = exp2(S' - lse'),  dP = dO V^T,
//   dS = P o (dP - Dq),  dV^T += dO^T P,  dK^T += Q^T dS,  dQ += dS K,
// five 32x32x32 products -- the query- and key-stationary kernel pair
// computes S' and dP twice, seven products.  S' and dP land with one key per
// lane (queries in the accumulator's register order), the layout dV and dK
// contract over; dQ contracts over keys, so dS is transposed through a
// per-wave LDS scratch before the dQ product.
//
// The dQ sum over key tiles runs as a chain instead of atomics (a 64-lane
// ds_add_f32 measured ~650 cycles on gfx950; global float atomics cost ~10 us
// at c1): at step t the wave of key tile j handles query tile i = j + t
// (causal; (j + t) mod nt otherwise), so the contributions to tile i arrive
// from key tiles i, i-1, ..., each one step after the previous.  A wave adds
// its dQ tile to the partial left in LDS by key tile j+1 (waiting on the
// tile's counter, which that wave set when it stored the partial), and the
// last contributor writes the finished rows to global memory.  Every wait is
// on a wave one step behind in the chain, so all of them end; they are
// bounded besides.  Each wave stages its own diagonal query tile (Q, dO
// rows, lse', Dq = dO . O) and flags it, so no workgroup-wide barrier follows
// the start.  The summation order is fixed: results are deterministic.
//
// One launch, no atomics, no workspace; the LDS footprint (154 KB at
// S = 256) allows one workgroup per CU, two waves per SIMD, and the causal
// key tiles j and nt-1-j share a SIMD (nt + 1 tiles per SIMD).
#pragma once

#include <atomic>
#include <type_traits>

#include "bwd_tiled.h"
#include "common.h"
#include "fa_common.h"
#include "kernels.h"

namespace hipgpt {
namespace bwd {
namespace bh {

constexpr int D = 32;
constexpr int NW = 8;          // waves; at most one key tile each
constexpr int MAXS = NW * BK;  // longest sequence
constexpr int RP = D + 4;      // pitch of the Q / dO rows
constexpr int XP = BK + 4;     // pitch of a wave's dS^T scratch ([key][query])
constexpr int PP = D + 8;      // pitch of the dQ partials: rows q and q+4 on disjoint banks
constexpr int CPR = D / 4;     // 16-byte chunks per row

constexpr int kSpinMax = 1 << 20;  // bound of a flag wait (~0.1 s)

// HBM bytes per s_memrealtime tick (10 ns) assumed by the staggered start.
constexpr unsigned long long kSlotDiv = 60000;

// LDS layout in floats for Sp = S rounded up to 32 rows.
struct Layout {
    int q, g, dqa, l2, dv, x, total;
};
__host__ __device__ constexpr Layout layout(int Sp) {
    return Layout{0,
                  Sp * RP,
                  2 * Sp * RP,
                  2 * Sp * RP + Sp * PP,
                  2 * Sp * RP + Sp * PP + Sp,
                  2 * Sp * RP + Sp * PP + 2 * Sp,
                  2 * Sp * RP + Sp * PP + 2 * Sp + NW * BK * XP};
}
constexpr int kMaxLdsBytes = layout(MAXS).total * 4;

// Wait until *flag >= v (another wave of the workgroup stores it with
// release order), for at most kSpinMax polls; an expiry is counted
// (note_wait_expired) for the host to see.
__device__ __forceinline__ void wait_ge(const int* flag, int v) {
    for (int n = 0; n < kSpinMax; ++n) {
        if (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= v) return;
        __builtin_amdgcn_s_sleep(1);
    }
    if ((threadIdx.x & 63) == 0) note_wait_expired();
}
__device__ __forceinline__ void set_flag(int* flag, int v) {
    __hip_atomic_store(flag, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Key of dQ product step s in lane half h (any bijection of the 32 keys
// works; this one puts the two halves' scratch rows 8 apart, on disjoint
// LDS banks).
__device__ __forceinline__ int dq_key(int s, int h) { return 16 * (s >> 3) + 8 * h + (s & 7); }

// Stored P of query tile i and key kj in the accumulator's order (register r
// <-> query i*32 + acc_key(r, h), lane <-> key kj) from the (b, h) slice
// `pr` of the [S][S] probs; keys past S read as zero through an
// out-of-range offset.  The buffer range check covers the vector offset (and
// the immediate) only, never the scalar offset: a whole tile in range puts
// each register's row offset in the scalar operand, the last tile of a ragged
// S (rows past S) folds it into the vector offset so those rows read as zero.
// A wave's 32 x 32 gradient block (key kj = row0 + c on lane (c, h),
// register r <-> dim acc_key(r, h)), times mul, stored as whole 128-byte rows
// through the wave's scratch X (pitch XP), non-temporally; rows past S are
// dropped.  X must be free: its earlier reads issued (a wave's LDS accesses
// run in order; the memory clobbers keep the compiler's order).
// Cache policy of the dQ row stores (whole rows already): non-temporal.
constexpr int kDqPolicy = 2;
__device__ __forceinline__ void store_rows_t(float* X, float* dst0, const floatx16& acc, float mul, int row0, int S,
                                             int64_t ts, int lane) {
    const int c = lane & 31, hf = lane >> 5;
    asm volatile("" ::: "memory");
#pragma unroll
    for (int g = 0; g < 4; ++g)
        *reinterpret_cast<floatx4*>(X + c * XP + 8 * g + 4 * hf) =
            floatx4{mul * acc[4 * g], mul * acc[4 * g + 1], mul * acc[4 * g + 2], mul * acc[4 * g + 3]};
    asm volatile("" ::: "memory");
    const int rr = lane >> 3, cc = 4 * (lane & 7);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int row = 8 * k + rr;
        const floatx4 v = *reinterpret_cast<const floatx4*>(X + row * XP + cc);
        if (row0 + row < S) __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(dst0 + (int64_t)row * ts + cc));
    }
    asm volatile("" ::: "memory");
}

// Stored-probs loads of the single-read kernels (each P element read once):
// non-temporal (c1 drop-in backward 52.2 -> 50.6 us cache-rotated).
constexpr int kPPolicy = 2;
__device__ __forceinline__ void load_p_tile(floatx16& pv, __amdgpu_buffer_rsrc_t pr, int i, int kj, bool kval, int hf,
                                            int S) {
    const int S4 = S * 4;
    const int vo = kval ? (i * BK + 4 * hf) * S4 + kj * 4 : 0x40000000;
    if (i * BK + BK <= S) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            pv[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pr, vo, (8 * (r >> 2) + (r & 3)) * S4, kPPolicy));
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            pv[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pr, vo + (8 * (r >> 2) + (r & 3)) * S4, 0, kPPolicy));
    }
}

template <bool CAUSAL>
__global__ __launch_bounds__(NW * 64) void bwd_bh_kernel(BwdArgs a) {
    const unsigned long long t_start = __builtin_amdgcn_s_memrealtime();
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ int simd_slots[NW];
    __shared__ int staged[NW];  // query tile t's rows are in LDS
    __shared__ int chain[NW];   // contributions summed into query tile t's dQ partial
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, hf = lane >> 5;
    const int bhi = blockIdx.x;
    const int b = bhi / a.H, h = bhi % a.H;
    const int S = a.S, nt = (S + BK - 1) / BK, Sp = nt * BK;
    const Layout L = layout(Sp);
    float* const Qr = lds + L.q;
    float* const Gr = lds + L.g;
    float* const DQA = lds + L.dqa;  // dQ partials [Sp][PP]
    float* const L2 = lds + L.l2;
    float* const DV = lds + L.dv;
    float* const X = lds + L.x + wave * BK * XP;
    const int64_t base = (int64_t)b * a.bs + (int64_t)h * a.hs;

    if (tid < NW) staged[tid] = chain[tid] = 0;
    // Key tile of this wave: SIMD s (ranks 2s, 2s+1) takes tiles s and
    // nt-1-s, so causal work pairs up to nt + 1 tiles per SIMD.  The rank's
    // barrier also publishes the cleared flags.
    const int sr = fa::simd_rank<NW>(simd_slots, wave, lane);
    const int s2 = sr >> 1;
    int kt = -1;
    if (s2 < (nt + 1) / 2) kt = (sr & 1) ? (nt - 1 - s2 > s2 ? nt - 1 - s2 : -1) : s2;
    if (kt < 0) return;

    // Causal: key tile kt first needs query tile kt + t at its step t, and the
    // wave of key tile 0 has the most steps.  Starting wave kt's loads kt
    // slots after the workgroup start (a slot: the time HBM takes to deliver
    // one key tile's rows for every resident workgroup, at ~6 TB/s) lets the
    // early key tiles' rows arrive first instead of every wave waiting for all
    // of them.  s_memrealtime counts 10 ns; the wait is at most 7 slots.
    // Only the first set of workgroups, which the device starts together,
    // loads in a burst; later ones start as slots free up and are not delayed.
    if (CAUSAL && kt > 0 && bhi < a.resident) {
        constexpr int kWaveBytes = 5 * BK * D * 4;  // Q, dO, O rows + K, V rows
        const unsigned long long slot = (unsigned long long)a.resident * kWaveBytes / kSlotDiv;
        const unsigned long long until = t_start + slot * kt;
        for (int n = 0; n < 4096 && __builtin_amdgcn_s_memrealtime() < until; ++n) __builtin_amdgcn_s_sleep(2);
    }

    // Stage query tile kt: Q and dO rows, and (recompute) Dq = dO . O and
    // lse' = lse log2 e (+inf past S: P = 0 there); and the wave's keys: K
    // pre-scaled to log2 units and V (B operands of S' and dP, lane (c, h)
    // holds dims 16h .. 16h+15 of key kj), K as the B operand of a product
    // over keys (step s: key dq_key(s, h), dim c), read back through the
    // scratch.  Every global load is issued before the
    // first use (one round trip); rows past S load as zero.
    const int kj = kt * BK + c;
    const bool kval = kj < S;
    float kr2[D / 2], vr[D / 2], kq[16];
    {
        RowLoader ql, gl, ol, kl, vl;
        ql.init(a.q + base, a.ts, S, D);
        gl.init(a.go + base, a.ts, S, D);
        ol.init(a.o + base, a.ts, S, D);
        kl.init(a.k + base, a.ts, S, D);
        vl.init(a.v + base, a.ts, S, D);
        constexpr int NK = BK * CPR / 64;
        floatx4 qv[NK], gv[NK], ov[NK], kv[D / 8], vv[D / 8];
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int f = lane + 64 * k;
            const int row = kt * BK + f / CPR, cc = f % CPR;
            qv[k] = ql.load(row, cc);
            gv[k] = gl.load(row, cc);
            ov[k] = ol.load(row, cc);
        }
#pragma unroll
        for (int s = 0; s < D / 8; ++s) {
            kv[s] = kl.load(kj, hf * (D / 8) + s);
            vv[s] = vl.load(kj, hf * (D / 8) + s);
        }
        const int ql2 = kt * BK + (lane & (BK - 1));
        const float lsev = ql2 < S ? a.lse[(int64_t)bhi * S + ql2] : 0.f;
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int f = lane + 64 * k;
            const int row = kt * BK + f / CPR, cc = f % CPR;
            *reinterpret_cast<floatx4*>(Qr + row * RP + 4 * cc) = qv[k];
            *reinterpret_cast<floatx4*>(Gr + row * RP + 4 * cc) = gv[k];
            float d = gv[k][0] * ov[k][0];
#pragma unroll
            for (int j = 1; j < 4; ++j) d = fmaf(gv[k][j], ov[k][j], d);
#pragma unroll
            for (int m = 1; m < CPR; m <<= 1) d += __shfl_xor(d, m);
            if (cc == 0) DV[row] = d;
        }
        if (lane < BK) L2[ql2] = ql2 < S ? lsev * kLog2e : kInf;
        const float qsc = a.scale * kLog2e;
#pragma unroll
        for (int s = 0; s < D / 8; ++s) {
            *reinterpret_cast<floatx4*>(X + c * XP + hf * (D / 2) + 4 * s) = kv[s];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                kr2[4 * s + j] = kv[s][j] * qsc;
                vr[4 * s + j] = vv[s][j];
            }
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) kq[s] = X[dq_key(s, hf) * XP + c];
    }
    set_flag(&staged[kt], 1);

    const bool kedge = kt * BK + BK > S;  // keys past S in this tile
    const int nsteps = CAUSAL ? nt - kt : nt;

    floatx16 accv, acck;  // dV^T, dK^T (unscaled): register r <-> dim acc_key(r, h), lane <-> key
#pragma unroll
    for (int r = 0; r < 16; ++r) accv[r] = acck[r] = 0.f;

    // dQ term of the job whose dS^T is in the scratch: A[query][key] = X[key][query]
    auto dq_term = [&]() {
        floatx16 aq;
#pragma unroll
        for (int r = 0; r < 16; ++r) aq[r] = 0.f;
#pragma unroll
        for (int s = 0; s < 16; ++s)
            aq = __builtin_amdgcn_mfma_f32_32x32x2f32(X[dq_key(s, hf) * XP + c], kq[s], aq, 0, 0, 0);
        return aq;
    };
    // dQ rows through a buffer resource ending at row S-1.  As for the P
    // loads of the stored-probs kernel, only the vector offset is range-checked: whole tiles use a scalar
    // row offset per register, the last tile of a ragged S puts it in the
    // vector offset so the stores of rows past S are dropped.
    const __amdgpu_buffer_rsrc_t dqr = __builtin_amdgcn_make_buffer_rsrc(
        a.dq + base, 0, (int)(((int64_t)(S - 1) * a.ts + D) * 4), kBufferFlags);
    const int row4 = a.ts * 4;
    // Chain step t of query tile i: register r <-> query i*32 + acc_key(r, h),
    // lane <-> dim c.
    auto chain_add = [&](floatx16 aq, int i, int t) {
        const int nc = CAUSAL ? i + 1 : nt;  // contributors of tile i
        float* const part = DQA + (i * BK + 4 * hf) * PP + c;
        if (t > 0) {
            wait_ge(&chain[i], t);
#pragma unroll
            for (int r = 0; r < 16; ++r) aq[r] += part[(8 * (r >> 2) + (r & 3)) * PP];
        }
        if (t == nc - 1) {
            const int vo = (i * BK + 4 * hf) * row4 + c * 4;
            if (i * BK + BK <= S) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(a.scale * aq[r]), dqr, vo,
                                                          (8 * (r >> 2) + (r & 3)) * row4, kDqPolicy);
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(a.scale * aq[r]), dqr,
                                                          vo + (8 * (r >> 2) + (r & 3)) * row4, 0, kDqPolicy);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) part[(8 * (r >> 2) + (r & 3)) * PP] = aq[r];
            set_flag(&chain[i], t + 1);
        }
    };
    // Job t (query tile i).  The previous job's dQ term is formed alongside
    // this job's S' and dP products (one basic block, so their MFMAs and LDS
    // reads interleave) and enters the chain after this job's dV / dK.
    int iprev = 0;
    auto job = [&](auto has_prev, int t) {
        constexpr bool HP = decltype(has_prev)::value;
        int i = kt + t;
        if (!CAUSAL && i >= nt) i -= nt;
        if (HP) wait_ge(&staged[i], 1);
        const float* qt = Qr + i * BK * RP;
        const float* gt = Gr + i * BK * RP;
        // The chains start from -lse' and -Dq, so they end at S' - lse' and
        // dP - Dq: P = exp2(first), dS = P * second.
        floatx16 sc, dp;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const floatx4 l4 = *reinterpret_cast<const floatx4*>(L2 + i * BK + 8 * g + 4 * hf);
            const floatx4 d4 = *reinterpret_cast<const floatx4*>(DV + i * BK + 8 * g + 4 * hf);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sc[4 * g + j] = -l4[j];
                dp[4 * g + j] = -d4[j];
            }
        }
        floatx16 p, ds;
        Tiles<D>::dchain(sc, qt, kr2, c, hf);  // S' - lse', register r <-> query i*32 + acc_key(r, h)
        Tiles<D>::dchain(dp, gt, vr, c, hf);  // dP - Dq
        floatx16 aq;
        if constexpr (HP) aq = dq_term();
        // masks: keys past S (last key tile) and, causally, keys past the
        // query on the diagonal job (t == 0)
        const bool edge = HP ? kedge : (kedge || CAUSAL);
        if (edge) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const bool vis = kval && (!CAUSAL || kj <= i * BK + acc_key(r, hf));
                p[r] = vis ? fast_exp2(sc[r]) : 0.f;
                ds[r] = p[r] * dp[r];
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                p[r] = fast_exp2(sc[r]);
                ds[r] = p[r] * dp[r];
            }
        }
        // dV^T += dO^T P, dK^T += Q^T dS: A[d][query] read from the row-major tiles
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int q = acc_key(r, hf);
            accv = __builtin_amdgcn_mfma_f32_32x32x2f32(gt[q * RP + c], p[r], accv, 0, 0, 0);
            acck = __builtin_amdgcn_mfma_f32_32x32x2f32(qt[q * RP + c], ds[r], acck, 0, 0, 0);
        }
        if constexpr (HP) chain_add(aq, iprev, t - 1);
        // this job's dS^T into the scratch ([key][query]; the previous job's
        // reads of it were issued above, and a wave's LDS accesses run in order)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<floatx4*>(X + c * XP + 8 * g + 4 * hf) =
                floatx4{ds[4 * g], ds[4 * g + 1], ds[4 * g + 2], ds[4 * g + 3]};
        iprev = i;
    };
    job(std::false_type{}, 0);
    for (int t = 1; t < nsteps; ++t) job(std::true_type{}, t);
    chain_add(dq_term(), iprev, nsteps - 1);

    // dV, dK through the wave's scratch (its last reads were issued above):
    // whole 128-byte rows, non-temporal
    store_rows_t(X, a.dv + base + (int64_t)(kt * BK) * a.ts, accv, 1.f, kt * BK, S, a.ts, lane);
    store_rows_t(X, a.dk + base + (int64_t)(kt * BK) * a.ts, acck, a.scale, kt * BK, S, a.ts, lane);
}

// ---------------------------------------------------------------------------
// Stored probs (the reference's contract; its drop-in call has no causal
// mask): every P tile is read from memory once.
//
// At step t every wave works on query tile t against its own key tile j, so
// the row sums Dq_t = sum_j rowsum(P_tj o dP_tj) complete with one
// workgroup barrier per step.  A wave forms dP_tj = dO_t V_j^T a step ahead,
// sums P o dP over its 32 keys (transposed through its LDS scratch) and
// publishes the 32 partial sums; after the barrier each wave adds the
// partials in key-tile order.  dS = P o (dP - Dq), dV^T += dO^T P and
// dK^T += Q^T dS then use the P tile still in registers.  dQ of query tile t
// is the sum of the waves' 32x32 terms dS_tj K_j: each wave leaves its term
// in a double-buffered LDS area and, after the next barrier, every wave adds
// the terms of four of the 32 rows in key-tile order and writes them.  Q and
// dO tiles stream through a three-slot LDS ring, staged by all threads two
// steps ahead.  Per step a wave runs 64 MFMAs (dP, dV, dK, dQ; the
// probs-free kernel above runs 80, as it rebuilds S') and waits on no flag.
// Causally the wave of key tile j has nothing to add for query tiles t < j
// (P = 0 there): it skips those steps' products and P reads, keeps its
// slots of the per-step sums at zero, and joins the barriers.
// All summation orders are fixed: results are deterministic.
namespace nc {
// LDS layout in floats.  The per-wave scratch and the ring come first: DS
// instructions take immediate offsets below 64 KB only, and those two areas
// take most of the accesses.
constexpr int TILE = BK * RP;  // one Q or dO tile, row-major with pitch RP
constexpr int SLOTS = 3;       // ring slots, each a Q tile then a dO tile
constexpr int XS = 0;          // per-wave scratch [NW][BK][XP]
constexpr int RING = XS + NW * BK * XP;
constexpr int PD = RING + SLOTS * 2 * TILE;  // partial row sums [2][NW][BK]
constexpr int DQP = PD + 2 * NW * BK;        // dQ terms [2][NW][BK][PP]
constexpr int TOTAL = DQP + 2 * NW * BK * PP;
constexpr int kLdsBytes = TOTAL * 4;
// The step's Dq sits in the scratch rows' pitch padding: query q at row q / 4,
// column BK + q % 4.
constexpr int DQCOL = BK;
static_assert(XP >= BK + 4, "room for the step's Dq in the scratch pitch");
static_assert(PD * 4 <= 65536, "scratch and ring within the DS immediate range");
static_assert(kLdsBytes <= 160 * 1024, "LDS of the single-read kernel");
static_assert(NW * 32 == BK * CPR, "one 16-byte chunk of a Q or dO tile per thread of half the workgroup");
}  // namespace nc

// Workgroup barrier that publishes LDS writes only: each wave waits for its
// own LDS accesses, not for its global loads in flight (a workgroup-scope
// fence, as in __syncthreads, would also wait for the prefetched P tiles and
// ring rows).  The memory clobber keeps the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// A per-lane LDS float offset the compiler cannot fold into constants: the
// accesses through it then carry their constant part as an immediate offset
// (below 64 KB) instead of a full address computed per access.
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

template <bool CAUSAL>
__global__ __launch_bounds__(NW * 64) void bwd_bh_probs_kernel(BwdArgs a) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, hf = lane >> 5;
    const int bhi = blockIdx.x;
    const int b = bhi / a.H, h = bhi % a.H;
    const int S = a.S, nt = (S + BK - 1) / BK;
    const int64_t base = (int64_t)b * a.bs + (int64_t)h * a.hs;
    const bool active = wave < nt;  // the wave owns key tile `wave`
    const int kj = wave * BK + c;
    const bool kval = kj < S;
    float* const X = lds + nc::XS + wave * BK * XP;

    // Q / dO ring: tile i sits in slot i % 3 (Q, then dO).  Waves 0-3 stage
    // the Q tile, waves 4-7 the dO tile, one 16-byte chunk per thread; rows
    // past S read as zero.  Tiles past the last (i < nt + 3) are staged too:
    // they read as zero, and their slot's tile i-3 has been read by then.
    RowLoader rl;
    rl.init((wave < NW / 2 ? a.q : a.go) + base, a.ts, S, D);
    const int sf = tid & (NW * 32 - 1);
    const int srow = sf / CPR, scc = sf % CPR;
    const int soff = (wave < NW / 2 ? 0 : nc::TILE) + srow * RP + 4 * scc;
    auto slot = [&](int i) { return lds + nc::RING + (i % nc::SLOTS) * 2 * nc::TILE; };
    auto ring_load = [&](int i) { return rl.load(i * BK + srow, scc); };
    auto ring_store = [&](int i, const floatx4& v) { *reinterpret_cast<floatx4*>(slot(i) + soff) = v; };

    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(a.probs) + (int64_t)bhi * S * S, 0, S * S * 4, kBufferFlags);

    // The wave's keys: V (B operand of dP, lane (c, h) holding dims
    // 16h .. 16h+15 of key kj) and K as the B operand of the dQ product over
    // keys (step s: key dq_key(s, h), dim c), read back through the scratch.
    // Every workgroup starts at once, so the first loads arrive as one burst
    // over the whole device: only what the first step needs is requested
    // before it (ring tiles 0 and 1, V, P of tile 0, K, in order of first
    // use); P of tile 1 and ring tile 2 follow once the first step runs.
    float vr[D / 2], kq[16];
    floatx16 p, pn;  // P of the step's query tile and of the next one
    floatx4 r0 = ring_load(0), r1 = ring_load(1);
    floatx4 kv[D / 8], vv[D / 8];
    RowLoader kl, vl;
    kl.init(a.k + base, a.ts, S, D);
    vl.init(a.v + base, a.ts, S, D);
    // Causal probs: query tiles before the wave's key tile (t < wave) hold
    // P = 0, so their tiles are neither read nor computed with; the wave's P
    // pipeline holds zeros there.
    const bool p0 = !CAUSAL || wave == 0, p1 = !CAUSAL || wave <= 1;
    if (active) {
#pragma unroll
        for (int s = 0; s < D / 8; ++s) vv[s] = vl.load(kj, hf * (D / 8) + s);
        if (p0) {
            load_p_tile(p, pr, 0, kj, kval, hf, S);
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = 0.f;
        }
#pragma unroll
        for (int s = 0; s < D / 8; ++s) kv[s] = kl.load(kj, hf * (D / 8) + s);
    }
    ring_store(0, r0);
    ring_store(1, r1);
    if (!active || CAUSAL) {
        // a wave past the last key tile (causal: every wave, whose first
        // steps contribute nothing) zeroes its partial-sum and dQ-term slots
        // once, so the sums over all NW waves need no selects
        lds[nc::PD + (hf * NW + wave) * BK + c] = 0.f;
#pragma unroll
        for (int k = 0; k < 2 * BK * (BK / 4) / 64; ++k) {
            const int f = lane + 64 * k;  // [parity][row][chunk of four dims]
            const int par = f / (BK * BK / 4), row = (f / (BK / 4)) % BK, c4 = f % (BK / 4);
            *reinterpret_cast<floatx4*>(lds + nc::DQP + ((par * NW + wave) * BK + row) * PP + 4 * c4) =
                floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }

    // Per-lane bases of the areas above 64 KB (constant parts as immediates).
    const float* const pdl = lds + opaque(nc::PD + c);                            // + (parity * NW + v) * BK
    float* const dqw = lds + opaque(nc::DQP + wave * BK * PP + 4 * hf * PP + c);  // + parity * NW*BK*PP + row * PP
    const int rrow = 4 * wave + (lane >> 4), rd2 = 2 * (lane & 15);
    const float* const dqr0 = lds + opaque(nc::DQP + rrow * PP + rd2);            // + v * BK*PP
    const float* const dqr1 = lds + opaque(nc::DQP + NW * BK * PP + rrow * PP + rd2);

    // dP = dO_i V_j^T of the dO tile `gt` (register r <-> query acc_key(r, h),
    // lane <-> key), the chain starting from zero.
    auto dp_tile = [&](const float* gt) {
        const float* rr = gt + c * RP + hf * (D / 2);
        floatx4 dv[D / 8];
#pragma unroll
        for (int j = 0; j < D / 8; ++j) dv[j] = *reinterpret_cast<const floatx4*>(rr + 4 * j);
        floatx16 acc = __builtin_amdgcn_mfma_f32_32x32x2f32(dv[0][0], vr[0], floatx16{}, 0, 0, 0);
#pragma unroll
        for (int k = 1; k < D / 2; ++k) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(dv[k >> 2][k & 3], vr[k], acc, 0, 0, 0);
        return acc;
    };
    // Row sums of P o dP of a query tile over this wave's keys into the PD
    // entry of parity PAR: the product is stored transposed ([key][query])
    // and lane (c, h) adds keys 16h .. 16h+15 of query c, the two halves
    // starting eight keys apart (disjoint banks); then the halves are added.
    auto partial = [&](auto par_tag, const floatx16& pv, const floatx16& dpv) {
        constexpr int PAR = decltype(par_tag)::value;
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<floatx4*>(X + c * XP + 8 * g + 4 * hf) =
                floatx4{pv[4 * g] * dpv[4 * g], pv[4 * g + 1] * dpv[4 * g + 1], pv[4 * g + 2] * dpv[4 * g + 2],
                        pv[4 * g + 3] * dpv[4 * g + 3]};
        const float* xa = X + (24 * hf) * XP + c;  // keys 24h + u, u < 8 (h = 1: 24 .. 31)
        const float* xb = X + (8 * hf) * XP + c;   // keys 8h + u, u >= 8 (h = 1: 16 .. 23)
        float s = 0.f;
#pragma unroll
        for (int u = 0; u < 8; ++u) s += xa[u * XP];
#pragma unroll
        for (int u = 8; u < 16; ++u) s += xb[u * XP];
        s += __shfl_xor(s, 32);
        if (hf == 0) lds[nc::PD + (PAR * NW + wave) * BK + c] = s;
    };

    lds_barrier();  // ring tiles 0 and 1

    floatx16 dp, dpn;  // dP of the step's query tile and of the next one
    if (active) {
#pragma unroll
        for (int s = 0; s < D / 8; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j) vr[4 * s + j] = vv[s][j];
        if (p0) {
            dp = dp_tile(slot(0) + nc::TILE);
            partial(std::integral_constant<int, 0>{}, p, dp);
        }
    }

    // dQ rows of query tile i (parity PAR): wave w adds rows 4w .. 4w+3 of the
    // waves' terms (two dims per lane) in key-tile order and writes them
    // through a buffer resource ending at row S-1 (rows past S are dropped).
    const __amdgpu_buffer_rsrc_t dqr = __builtin_amdgcn_make_buffer_rsrc(
        a.dq + base, 0, (int)(((int64_t)(S - 1) * a.ts + D) * 4), kBufferFlags);
    const int row4 = a.ts * 4;
    auto reduce_dq = [&](auto par_tag, int i) {
        constexpr int PAR = decltype(par_tag)::value;
        const float* src = PAR ? dqr1 : dqr0;
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int v = 0; v < NW; ++v) {  // terms past the last key tile are zeros
            const float2 x = *reinterpret_cast<const float2*>(src + v * BK * PP);
            s0 += x.x;
            s1 += x.y;
        }
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(a.scale * s0), __float_as_uint(a.scale * s1)}, dqr,
                                              (i * BK + rrow) * row4 + rd2 * 4, 0, kDqPolicy);
    };

    floatx16 accv, acck;  // dV^T, dK^T (unscaled): register r <-> dim acc_key(r, h), lane <-> key
#pragma unroll
    for (int r = 0; r < 16; ++r) accv[r] = acck[r] = 0.f;
    lds_barrier();  // step 0's partial row sums
    floatx4 rn = ring_load(2);
    if (active) {
        if (nt > 1) {
            if (p1) {
                load_p_tile(pn, pr, 1, kj, kval, hf, S);
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) pn[r] = 0.f;
            }
        }
        // K through the scratch (the partial sums' reads of it are done)
#pragma unroll
        for (int s = 0; s < D / 8; ++s) *reinterpret_cast<floatx4*>(X + c * XP + hf * (D / 2) + 4 * s) = kv[s];
#pragma unroll
        for (int s = 0; s < 16; ++s) kq[s] = X[dq_key(s, hf) * XP + c];
    }

    // One step of an active wave on query tile t (t % 2 == PAR): pc / dc hold
    // P / dP of tile t, pnx P of tile t+1; a step with a successor (LAST
    // false) forms dnx = dP of tile t+1 and its partial row sums, and loads P
    // of tile t+2 into pc (the last tile again past the end).  Steps
    // alternate the buffers' roles, so no registers are copied.
    auto step = [&](auto last_tag, auto par_tag, auto early_tag, int t, floatx16& pc, floatx16& pnx, floatx16& dc,
                    floatx16& dnx) {
        constexpr bool LAST = decltype(last_tag)::value;
        constexpr int PAR = decltype(par_tag)::value;
        constexpr bool EARLY = decltype(early_tag)::value;
        const float* qt = slot(t);
        const float* gt = qt + nc::TILE;
        if constexpr (EARLY && !LAST) dnx = dp_tile(slot(t + 1) + nc::TILE);
        // Dq of query tile t (lane: query c): the partials in key-tile order
        // (zeros past the last key tile), kept in the scratch's padding for
        // the register-order reads below
        float dsum = 0.f;
#pragma unroll
        for (int v = 0; v < NW; ++v) dsum += pdl[(PAR * NW + v) * BK];
        if (hf == 0) X[(c >> 2) * XP + nc::DQCOL + (c & 3)] = dsum;
        // dV^T += dO^T P: A[d][query] read from the row-major dO tile
#pragma unroll
        for (int r = 0; r < 16; ++r)
            accv = __builtin_amdgcn_mfma_f32_32x32x2f32(gt[acc_key(r, hf) * RP + c], pc[r], accv, 0, 0, 0);
        floatx16 ds;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const floatx4 d4 = *reinterpret_cast<const floatx4*>(X + (2 * g + hf) * XP + nc::DQCOL);
#pragma unroll
            for (int j = 0; j < 4; ++j) ds[4 * g + j] = pc[4 * g + j] * (dc[4 * g + j] - d4[j]);
        }
        // dK^T += Q^T dS
#pragma unroll
        for (int r = 0; r < 16; ++r)
            acck = __builtin_amdgcn_mfma_f32_32x32x2f32(qt[acc_key(r, hf) * RP + c], ds[r], acck, 0, 0, 0);
        // dQ term dS K: dS^T through the scratch ([key][query]), A[query][key] = X[key][query]
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<floatx4*>(X + c * XP + 8 * g + 4 * hf) =
                floatx4{ds[4 * g], ds[4 * g + 1], ds[4 * g + 2], ds[4 * g + 3]};
        floatx16 aq = __builtin_amdgcn_mfma_f32_32x32x2f32(X[dq_key(0, hf) * XP + c], kq[0], floatx16{}, 0, 0, 0);
#pragma unroll
        for (int s = 1; s < 16; ++s)
            aq = __builtin_amdgcn_mfma_f32_32x32x2f32(X[dq_key(s, hf) * XP + c], kq[s], aq, 0, 0, 0);
        if constexpr (!LAST) {
            // the next query tile: dP, the partial row sums, and P two tiles ahead
            if constexpr (!EARLY) dnx = dp_tile(slot(t + 1) + nc::TILE);
            load_p_tile(pc, pr, t + 2 < nt ? t + 2 : nt - 1, kj, kval, hf, S);
            partial(std::integral_constant<int, 1 - PAR>{}, pnx, dnx);
        }
        // this wave's dQ term of query tile t (register r <-> query acc_key(r, h), lane <-> dim c)
#pragma unroll
        for (int r = 0; r < 16; ++r) dqw[PAR * NW * BK * PP + (8 * (r >> 2) + (r & 3)) * PP] = aq[r];
    };
    // Causal: the step of a wave whose keys all follow query tile t.  Its
    // terms are zero (the slots hold zeros); it keeps the P pipeline (P of
    // tile t+2, zero while that tile is still before the wave's keys) and, one
    // step before its first tile, forms that tile's dP and partial row sums.
    auto idle_step = [&](auto par_tag, int t, floatx16& pc, floatx16& pnx, floatx16& dnx) {
        constexpr int PAR = decltype(par_tag)::value;
        if (t + 1 == wave) {
            dnx = dp_tile(slot(t + 1) + nc::TILE);
            partial(std::integral_constant<int, 1 - PAR>{}, pnx, dnx);
        }
        if (t + 2 >= wave) {
            load_p_tile(pc, pr, t + 2 < nt ? t + 2 : nt - 1, kj, kval, hf, S);
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) pc[r] = 0.f;
        }
    };
    auto run_step = [&](auto last_tag, auto par_tag, int t, floatx16& pc, floatx16& pnx, floatx16& dc, floatx16& dnx) {
        if (!active) return;
        if (!CAUSAL || t >= wave) {
            // unmasked: the waves of the upper half form the next tile's dP
            // first, so each SIMD's two waves (w, w + 4) reach their
            // matrix-free stretches at different times (c1 drop-in 50.5 ->
            // 49.9 us; the causal instance would exceed its registers)
            if (!CAUSAL && wave >= NW / 2)
                step(last_tag, par_tag, std::integral_constant<bool, !CAUSAL>{}, t, pc, pnx, dc, dnx);
            else
                step(last_tag, par_tag, std::false_type{}, t, pc, pnx, dc, dnx);
        } else
            idle_step(par_tag, t, pc, pnx, dnx);  // t < wave <= nt - 1: never the last step
    };
    // Every wave after its step on tile t: the dQ rows of tile t-1, the ring,
    // the barrier.
    auto finish = [&](auto par_tag, int t) {
        constexpr int PAR = decltype(par_tag)::value;
        if (t > 0) reduce_dq(std::integral_constant<int, 1 - PAR>{}, t - 1);
        ring_store(t + 2, rn);  // its slot held tile t-1, last read before the previous barrier
        rn = ring_load(t + 3);
        lds_barrier();
    };
    using Even = std::integral_constant<int, 0>;
    using Odd = std::integral_constant<int, 1>;
    int t = 0;
    for (; t + 2 < nt; t += 2) {
        run_step(std::false_type{}, Even{}, t, p, pn, dp, dpn);
        finish(Even{}, t);
        run_step(std::false_type{}, Odd{}, t + 1, pn, p, dpn, dp);
        finish(Odd{}, t + 1);
    }
    if (t + 1 < nt) {
        run_step(std::false_type{}, Even{}, t, p, pn, dp, dpn);
        finish(Even{}, t);
        run_step(std::true_type{}, Odd{}, t + 1, pn, p, dpn, dp);
        finish(Odd{}, t + 1);
        reduce_dq(Odd{}, t + 1);
    } else {
        run_step(std::true_type{}, Even{}, t, p, pn, dp, dpn);
        finish(Even{}, t);
        reduce_dq(Even{}, t);
    }

    if (active) {
        store_rows_t(X, a.dv + base + (int64_t)(wave * BK) * a.ts, accv, 1.f, wave * BK, S, a.ts, lane);
        store_rows_t(X, a.dk + base + (int64_t)(wave * BK) * a.ts, acck, a.scale, wave * BK, S, a.ts, lane);
    }
}

}  // namespace bh

// D = 32, S <= 256 and the tiled kernels' layout conditions (checked by the
// caller: bwd_tiled_ok).  Stored probs are read as single floats, so there
// is no condition on S or on the probs' alignment.
inline bool bh_ok(const BwdArgs& a) { return a.D == bh::D && a.S >= 1 && a.S <= bh::MAXS; }

// Raise a kernel's dynamic-LDS limit once per device (bit d of attr_set).
inline hipError_t raise_lds_limit(const void* kern, int bytes, std::atomic<unsigned long long>& attr_set) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const unsigned long long bit = (dev >= 0 && dev < 64) ? 1ull << dev : 0ull;
    if (!bit || !(attr_set.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess) return e;
        attr_set.fetch_or(bit, std::memory_order_release);
    }
    return hipSuccess;
}

template <bool CAUSAL>
hipError_t launch_bh_mode(const BwdArgs& a, hipStream_t s) {
    const int64_t grid = (int64_t)a.B * a.H;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    auto kern = bh::bwd_bh_kernel<CAUSAL>;
    static std::atomic<unsigned long long> attr_set{0};
    hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(kern), bh::kMaxLdsBytes, attr_set);
    if (e != hipSuccess) return e;
    const int Sp = (a.S + BK - 1) / BK * BK;
    const size_t lds = (size_t)bh::layout(Sp).total * 4;
    BwdArgs args = a;
    static ResidentSlots cache[bh::NW];  // per LDS footprint: Sp / 32 - 1
    const int slots = cache[Sp / BK - 1].get(reinterpret_cast<const void*>(kern), bh::NW * 64, lds);
    args.resident = (int)(grid < slots ? grid : slots);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(bh::NW * 64), lds, s, args);
    return hipGetLastError();
}

template <bool CAUSAL>
hipError_t launch_bh_probs_mode(const BwdArgs& a, hipStream_t s) {
    const int64_t grid = (int64_t)a.B * a.H;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    static std::atomic<unsigned long long> attr_set{0};
    auto kern = bh::bwd_bh_probs_kernel<CAUSAL>;
    hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(kern), bh::nc::kLdsBytes, attr_set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(bh::NW * 64), bh::nc::kLdsBytes, s, a);
    return hipGetLastError();
}

inline hipError_t launch_bh_probs(const BwdArgs& a, hipStream_t s) {
    return a.causal ? launch_bh_probs_mode<true>(a, s) : launch_bh_probs_mode<false>(a, s);
}

inline hipError_t launch_bh(const BwdArgs& a, hipStream_t s) {
    // stored probs: the single-read kernel
    if (a.probs) return launch_bh_probs(a, s);
    return a.causal ? launch_bh_mode<true>(a, s) : launch_bh_mode<false>(a, s);
}

}  // namespace bwd
}  // namespace hipgpt
