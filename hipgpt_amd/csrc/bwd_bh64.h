// bwd_bh64.h -- attention backward for head dim 64 and S <= 256 with one
// workgroup per (b, h): with stored probs, every P tile read from memory once
// (HipGPT's drop-in backward, src/hip_kernels.cpp:1159-1272, at E / H = 64 --
// the c2 shape, E = 512, H = 8 -- and the causal extended call), or from the
// forward's O and row log-sum-exp with P rebuilt (the probs-free pair).
//
// The step structure follows bwd_bh_probs_kernel (bwd_bh.h): at step t every
// wave works on query tile t against its own key tile j (K_j and V_j in
// registers), Dq_t = sum_j rowsum(P_tj o dP_tj) is completed from the waves'
// published partial sums, and dQ_t is the fixed-order sum of the waves'
// 32 x 64 terms dS_tj K_j in LDS.  At D = 64 the per-wave state (K and V as
// MFMA operands, dV^T and dK^T as two 32x32 blocks each) takes 128 registers,
// so dP of the next tile is not held across steps: each step forms dP_tj,
// publishes the partial sums, and a mid-step barrier completes Dq before dS.
// The same barrier orders the single buffer of dQ terms (the previous tile's
// rows are summed before it, this tile's terms are stored after it), and Q /
// dO need only a two-slot ring.  Per step a wave runs 128 MFMAs (dP, dV, dK,
// and dQ in two 32-dim blocks).  Causally the wave of key tile j skips the
// steps t < j and loads no P above the diagonal; every wave's partial-sum
// and dQ-term slots start at zero, so the fixed-order sums need no masks.
// All summation orders are fixed: results are deterministic.
//
// LSE (probs-free): Dq_i = dO_i . O_i needs no sweep over the keys, so each
// wave computes it, with lse' = lse log2 e, for the rows of its own query
// tile into an LDS table before the first step; no partial sums are formed.
// Each step rebuilds P = exp2(S' - lse') from S' = (c log2 e) Q K^T (K
// pre-scaled in registers; masks on the causal diagonal and on keys past S
// only), the S' and dP chains starting from -lse' and -Dq, so P = exp2(S'
// chain) and dS = P * (dP chain).  160 MFMAs per wave and step; the
// mid-step barrier only orders the single buffer of dQ terms.
#pragma once

#include "bwd_bh.h"

namespace hipgpt {
namespace bwd {
namespace bh {

namespace p64 {
constexpr int DK = 64;
constexpr int NB = DK / 32;     // 32-wide head-dim blocks
constexpr int RPd = DK + 4;     // pitch of the Q / dO ring rows
constexpr int CPRd = DK / 4;    // 16-byte chunks per row
constexpr int TILE = BK * RPd;  // one Q or dO tile
constexpr int SLOTS = 2;        // ring slots, each a Q tile then a dO tile
constexpr int PPd = DK + 8;     // pitch of a dQ term's rows: rows q and q+4 on disjoint banks
// LDS layout in floats (the per-wave scratch first: most accesses, and DS
// immediate offsets reach 64 KB only)
constexpr int XS = 0;                        // per-wave scratch [NW][BK][XP]
constexpr int RING = XS + NW * BK * XP;
constexpr int PD = RING + SLOTS * 2 * TILE;  // partial row sums [2][NW][BK]; LSE: lse' and Dq [2][MAXS]
constexpr int DQP = PD + 2 * NW * BK;        // dQ terms [NW][BK][PPd]
constexpr int TOTAL = DQP + NW * BK * PPd;
constexpr int kLdsBytes = TOTAL * 4;
constexpr int DQCOL = BK;  // the step's Dq in the scratch rows' pitch padding
static_assert(XP >= BK + 4, "room for the step's Dq in the scratch pitch");
static_assert(NW * BK == MAXS, "the LSE mode's lse' and Dq tables fit the partial-sum slots");
static_assert(kLdsBytes <= 160 * 1024, "LDS of the D = 64 single-read kernel");
static_assert(BK * CPRd == NW * 64, "one 16-byte chunk of each of Q and dO per thread and tile");
}  // namespace p64

template <bool CAUSAL, bool LSE>
__global__ __launch_bounds__(NW * 64) void bwd_bh64_kernel(BwdArgs a) {
    using namespace p64;
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
    float* const X = lds + XS + wave * BK * XP;
    // does the wave's key tile meet query tile i (causally: from its diagonal on)
    auto meets = [&](int i) { return active && (!CAUSAL || wave <= i); };

    // Q / dO ring: tile i sits in slot i % 2 (Q, then dO); each thread stages
    // one 16-byte chunk of each per tile, rows past S reading as zero.  Tile
    // i+1 is stored during step i (its slot's tile i-1 was last read before
    // the previous barrier) from registers loaded a step earlier.
    RowLoader rq, rg;
    rq.init(a.q + base, a.ts, S, DK);
    rg.init(a.go + base, a.ts, S, DK);
    const int srow = tid / CPRd, scc = tid % CPRd;
    const int soff = srow * RPd + 4 * scc;
    auto slot = [&](int i) { return lds + RING + (i & 1) * 2 * TILE; };
    struct Stage {
        floatx4 q, g;
    };
    auto ring_load = [&](int i) { return Stage{rq.load(i * BK + srow, scc), rg.load(i * BK + srow, scc)}; };
    auto ring_store = [&](int i, const Stage& st) {
        float* const sl = slot(i);
        *reinterpret_cast<floatx4*>(sl + soff) = st.q;
        *reinterpret_cast<floatx4*>(sl + TILE + soff) = st.g;
    };

    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        LSE ? nullptr : const_cast<float*>(a.probs) + (int64_t)bhi * S * S, 0, LSE ? 0 : S * S * 4, kBufferFlags);

    // The wave's keys: V (B operand of dP, lane (c, h) holding dims
    // 32h .. 32h+31 of key kj), with LSE also K pre-scaled by c log2 e (B
    // operand of S', the same layout), and K as the B operand of the dQ
    // product over keys (block n, step s: key dq_key(s, h), dim 32n + c),
    // read back through the scratch.  Only what the first step needs is
    // requested before it.
    float vr[DK / 2], kq[NB][16], kr[LSE ? DK / 2 : 1];
    floatx16 p, pn;  // stored probs: P of the step's query tile and of the next one
    const Stage r0 = ring_load(0);
    Stage rn = ring_load(1);
    floatx4 kv[DK / 8], vv[DK / 8];
    RowLoader kl, vl;
    kl.init(a.k + base, a.ts, S, DK);
    vl.init(a.v + base, a.ts, S, DK);
    if (active) {
#pragma unroll
        for (int s = 0; s < DK / 8; ++s) vv[s] = vl.load(kj, hf * (DK / 8) + s);
        if (!LSE && meets(0)) load_p_tile(p, pr, 0, kj, kval, hf, S);
#pragma unroll
        for (int s = 0; s < DK / 8; ++s) kv[s] = kl.load(kj, hf * (DK / 8) + s);
    }
    ring_store(0, r0);
    if constexpr (LSE) {
        // the rows of query tile `wave`: lse' = lse log2 e (+inf past S, so P
        // = 0 there) and Dq = dO . O, lane (c, h) summing dims 32h .. 32h+31
        // of row c; tables [S] at PD (lse') and PD + MAXS (Dq)
        if (active) {
            RowLoader ol, gl;
            ol.init(a.o + base, a.ts, S, DK);
            gl.init(a.go + base, a.ts, S, DK);
            const int row = wave * BK + c;
            const float lsev = row < S ? a.lse[(int64_t)bhi * S + row] : 0.f;
            float d = 0.f;
#pragma unroll
            for (int s2 = 0; s2 < DK / 8; ++s2) {
                const floatx4 o4 = ol.load(row, hf * (DK / 8) + s2), g4 = gl.load(row, hf * (DK / 8) + s2);
#pragma unroll
                for (int e = 0; e < 4; ++e) d = fmaf(g4[e], o4[e], d);
            }
            d += __shfl_xor(d, 32);
            if (hf == 0) {
                lds[PD + row] = row < S ? lsev * kLog2e : kInf;
                lds[PD + MAXS + row] = d;
            }
        }
    } else {
        // every wave's partial-sum slots start at zero: waves past the last
        // key tile, and causally before their diagonal, leave them so
        lds[PD + (hf * NW + wave) * BK + c] = 0.f;
    }
    // the same for the dQ-term slots
#pragma unroll
    for (int k = 0; k < BK * (DK / 4) / 64; ++k) {
        const int f = lane + 64 * k;  // [row][chunk of four dims]
        *reinterpret_cast<floatx4*>(lds + DQP + (wave * BK + f / (DK / 4)) * PPd + 4 * (f % (DK / 4))) =
            floatx4{0.f, 0.f, 0.f, 0.f};
    }

    // Per-lane bases of the areas past the scratch (constant parts as immediates).
    const float* const pdl = lds + opaque(PD + c);                               // + (parity * NW + v) * BK
    float* const dqw = lds + opaque(DQP + wave * BK * PPd + 4 * hf * PPd + c);  // + row * PPd + 32n
    const int rrow = 4 * wave + (lane >> 4), rdd = 4 * (lane & 15);
    const float* const dqr0 = lds + opaque(DQP + rrow * PPd + rdd);  // + v * BK*PPd

    // dP = dO_i V_j^T of the dO tile `gt` (register r <-> query acc_key(r, h),
    // lane <-> key), 16 dims of the lane's row at a time.
    auto dp_tile = [&](const float* gt) {
        const float* rr = gt + c * RPd + hf * (DK / 2);
        floatx16 acc;
#pragma unroll
        for (int hb = 0; hb < DK / 32; ++hb) {
            floatx4 dv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) dv[j] = *reinterpret_cast<const floatx4*>(rr + 16 * hb + 4 * j);
#pragma unroll
            for (int k = 0; k < 16; ++k)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(dv[k >> 2][k & 3], vr[16 * hb + k],
                                                           (hb | k) ? acc : floatx16{}, 0, 0, 0);
        }
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
        asm volatile("" ::: "memory");  // other lanes' writes (see the K transposition)
        const float* xa = X + (24 * hf) * XP + c;  // keys 24h + u, u < 8 (h = 1: 24 .. 31)
        const float* xb = X + (8 * hf) * XP + c;   // keys 8h + u, u >= 8 (h = 1: 16 .. 23)
        float s = 0.f;
#pragma unroll
        for (int u = 0; u < 8; ++u) s += xa[u * XP];
#pragma unroll
        for (int u = 8; u < 16; ++u) s += xb[u * XP];
        s += __shfl_xor(s, 32);
        if (hf == 0) lds[PD + (PAR * NW + wave) * BK + c] = s;
    };
    // dQ rows of query tile i: wave w adds rows 4w .. 4w+3 of the waves' terms
    // (four dims per lane) in key-tile order and writes them through a buffer
    // resource ending at row S-1 (rows past S are dropped).
    const __amdgpu_buffer_rsrc_t dqr = __builtin_amdgcn_make_buffer_rsrc(
        a.dq + base, 0, (int)(((int64_t)(S - 1) * a.ts + DK) * 4), kBufferFlags);
    const int row4 = a.ts * 4;
    auto reduce_dq = [&](int i) {
        floatx4 sm = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int v = 0; v < NW; ++v) {
            const floatx4 x = *reinterpret_cast<const floatx4*>(dqr0 + v * BK * PPd);
#pragma unroll
            for (int e = 0; e < 4; ++e) sm[e] += x[e];
        }
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(a.scale * sm[0]), __float_as_uint(a.scale * sm[1]),
                                                     __float_as_uint(a.scale * sm[2]), __float_as_uint(a.scale * sm[3])},
                                               dqr, (i * BK + rrow) * row4 + rdd * 4, 0, kDqPolicy);
    };

    lds_barrier();  // ring tile 0, the zeroed slots

    floatx16 accv[NB], acck[NB];  // dV^T, dK^T (unscaled): block n register r <-> dim 32n + acc_key(r, h), lane <-> key
#pragma unroll
    for (int n = 0; n < NB; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) accv[n][r] = acck[n][r] = 0.f;
    if (active) {
#pragma unroll
        for (int s = 0; s < DK / 8; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                vr[4 * s + j] = vv[s][j];
                if constexpr (LSE) kr[4 * s + j] = kv[s][j] * (a.scale * kLog2e);
            }
        if (!LSE && nt > 1 && meets(1)) load_p_tile(pn, pr, 1, kj, kval, hf, S);
        // K through the scratch, one 32-dim block at a time: lanes of half n
        // hold dims 32n .. 32n+31.  The lanes of the other half read what
        // these lanes wrote: a wave's LDS accesses run in order, and the
        // memory clobber keeps the compiler from reusing the values those
        // lanes read from the same addresses for the previous block.
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            if (hf == n)
#pragma unroll
                for (int s = 0; s < DK / 8; ++s) *reinterpret_cast<floatx4*>(X + c * XP + 4 * s) = kv[s];
            asm volatile("" ::: "memory");
#pragma unroll
            for (int s = 0; s < 16; ++s) kq[n][s] = X[dq_key(s, hf) * XP + c];
        }
    }

    // A chain over the head dim: acc[m = row c of `rt`][n = key c] += sum_d
    // rt[c][d] bv[d], lane (c, h) taking d = 32h .. 32h+31 (16 at a time).
    auto chain = [&](const float* rt, const float (&bv)[DK / 2], floatx16 acc) {
        const float* rr = rt + c * RPd + hf * (DK / 2);
#pragma unroll
        for (int hb = 0; hb < DK / 32; ++hb) {
            floatx4 dv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) dv[j] = *reinterpret_cast<const floatx4*>(rr + 16 * hb + 4 * j);
#pragma unroll
            for (int k = 0; k < 16; ++k) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(dv[k >> 2][k & 3], bv[16 * hb + k], acc, 0, 0, 0);
        }
        return acc;
    };
    // dV^T += dO^T P: A[d][query] read from the row-major dO tile
    auto grad_v = [&](const float* gt, const floatx16& pv) {
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                accv[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(gt[acc_key(r, hf) * RPd + 32 * n + c], pv[r], accv[n], 0, 0, 0);
    };
    // dK^T += Q^T dS, then the dQ term dS K: dS^T through the scratch
    // ([key][query]), one 32-dim block at a time, each stored as it completes
    // (register r <-> query acc_key(r, h), lane <-> dim 32n + c)
    auto grad_kq = [&](const float* qt, const floatx16& ds) {
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                acck[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(qt[acc_key(r, hf) * RPd + 32 * n + c], ds[r], acck[n], 0, 0, 0);
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<floatx4*>(X + c * XP + 8 * g + 4 * hf) = floatx4{ds[4 * g], ds[4 * g + 1], ds[4 * g + 2], ds[4 * g + 3]};
        asm volatile("" ::: "memory");
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            floatx16 aq = __builtin_amdgcn_mfma_f32_32x32x2f32(X[dq_key(0, hf) * XP + c], kq[n][0], floatx16{}, 0, 0, 0);
#pragma unroll
            for (int s = 1; s < 16; ++s)
                aq = __builtin_amdgcn_mfma_f32_32x32x2f32(X[dq_key(s, hf) * XP + c], kq[n][s], aq, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) dqw[(8 * (r >> 2) + (r & 3)) * PPd + 32 * n] = aq[r];
        }
    };
    const bool kedge = wave * BK + BK > S;  // keys past S in this wave's tile

    // Step t (t % 2 == PAR) of every wave.  Stored probs: pc holds P of tile
    // t, the other buffer P of tile t+1 (requested a step ago); P of tile t+2
    // goes into pc once dS is formed, so the two buffers alternate roles and
    // nothing is copied.  LSE: P is rebuilt, pc unused.
    auto step = [&](auto par_tag, int t, floatx16& pc) {
        constexpr int PAR = decltype(par_tag)::value;
        const bool cur = meets(t);
        const float* qt = slot(t);
        const float* gt = qt + TILE;
        // the dQ rows of tile t-1 (its terms were published by the last barrier)
        if (t > 0) reduce_dq(t - 1);
        if constexpr (LSE) {
            lds_barrier();  // every wave has read the dQ terms of tile t-1
            if (cur) {
                // S' - lse' and dP - Dq, register r <-> query t*32 + acc_key(r, h), lane <-> key
                floatx16 sc, dpc;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const floatx4 l4 = *reinterpret_cast<const floatx4*>(lds + PD + t * BK + 8 * g + 4 * hf);
                    const floatx4 d4 = *reinterpret_cast<const floatx4*>(lds + PD + MAXS + t * BK + 8 * g + 4 * hf);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        sc[4 * g + j] = -l4[j];
                        dpc[4 * g + j] = -d4[j];
                    }
                }
                sc = chain(qt, kr, sc);
                dpc = chain(gt, vr, dpc);
                floatx16 pv, ds;
                if (kedge || (CAUSAL && t == wave)) {  // keys past S, the causal diagonal
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const bool vis = kval && (!CAUSAL || kj <= t * BK + acc_key(r, hf));
                        pv[r] = vis ? fast_exp2(sc[r]) : 0.f;
                        ds[r] = pv[r] * dpc[r];
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        pv[r] = fast_exp2(sc[r]);
                        ds[r] = pv[r] * dpc[r];
                    }
                }
                grad_v(gt, pv);
                grad_kq(qt, ds);
            }
        } else {
            // dP of tile t and its partial row sums
            floatx16 dp;
            if (cur) {
                dp = dp_tile(gt);
                partial(std::integral_constant<int, PAR>{}, pc, dp);
            }
            lds_barrier();  // the partial sums of tile t; every wave has read the dQ terms of tile t-1
            if (cur) {
                // Dq of query tile t (lane: query c): the partials in key-tile
                // order, kept in the scratch's padding for the register-order reads
                float dsum = 0.f;
#pragma unroll
                for (int v = 0; v < NW; ++v) dsum += pdl[(PAR * NW + v) * BK];
                if (hf == 0) X[(c >> 2) * XP + DQCOL + (c & 3)] = dsum;
                asm volatile("" ::: "memory");
                // (written out here: through grad_v and grad_kq this branch
                // spills two registers at 256 VGPRs)
#pragma unroll
                for (int n = 0; n < NB; ++n)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        accv[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(gt[acc_key(r, hf) * RPd + 32 * n + c], pc[r],
                                                                       accv[n], 0, 0, 0);
                floatx16 ds;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const floatx4 d4 = *reinterpret_cast<const floatx4*>(X + (2 * g + hf) * XP + DQCOL);
#pragma unroll
                    for (int j = 0; j < 4; ++j) ds[4 * g + j] = pc[4 * g + j] * (dp[4 * g + j] - d4[j]);
                }
                if (t + 2 < nt) load_p_tile(pc, pr, t + 2, kj, kval, hf, S);
#pragma unroll
                for (int n = 0; n < NB; ++n)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        acck[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(qt[acc_key(r, hf) * RPd + 32 * n + c], ds[r],
                                                                       acck[n], 0, 0, 0);
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    *reinterpret_cast<floatx4*>(X + c * XP + 8 * g + 4 * hf) =
                        floatx4{ds[4 * g], ds[4 * g + 1], ds[4 * g + 2], ds[4 * g + 3]};
                asm volatile("" ::: "memory");
#pragma unroll
                for (int n = 0; n < NB; ++n) {
                    floatx16 aq =
                        __builtin_amdgcn_mfma_f32_32x32x2f32(X[dq_key(0, hf) * XP + c], kq[n][0], floatx16{}, 0, 0, 0);
#pragma unroll
                    for (int s = 1; s < 16; ++s)
                        aq = __builtin_amdgcn_mfma_f32_32x32x2f32(X[dq_key(s, hf) * XP + c], kq[n][s], aq, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) dqw[(8 * (r >> 2) + (r & 3)) * PPd + 32 * n] = aq[r];
                }
            } else if (t + 2 < nt && meets(t + 2)) {
                load_p_tile(pc, pr, t + 2, kj, kval, hf, S);  // causally: the wave's first tile
            }
        }
        ring_store(t + 1, rn);
        rn = ring_load(t + 2);
        lds_barrier();  // ring tile t+1, this step's dQ terms
    };
    using Even = std::integral_constant<int, 0>;
    using Odd = std::integral_constant<int, 1>;
    int t = 0;
    for (; t + 1 < nt; t += 2) {
        step(Even{}, t, p);
        step(Odd{}, t + 1, pn);
    }
    if (t < nt) step(Even{}, t, p);
    reduce_dq(nt - 1);

    if (active) {
        // dV, dK through the wave's scratch, one 32-dim block at a time: whole
        // 128-byte row segments, non-temporal (the scratch's last reads, the
        // dQ term's operands, were issued before the closing barrier)
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            store_rows_t(X, a.dv + base + (int64_t)(wave * BK) * a.ts + 32 * n, accv[n], 1.f, wave * BK, S, a.ts, lane);
            store_rows_t(X, a.dk + base + (int64_t)(wave * BK) * a.ts + 32 * n, acck[n], a.scale, wave * BK, S, a.ts,
                         lane);
        }
    }
}

}  // namespace bh

// D = 64 (causal or not), S <= 256, and the tiled kernels' layout conditions
// (checked by the caller).  Stored probs are read as single floats, so there
// is no condition on S or on the probs' alignment; without them the forward's
// O and lse are required (the caller checks that too).
inline bool bh_probs64_ok(const BwdArgs& a) {
    return a.probs && a.D == bh::p64::DK && a.S >= 1 && a.S <= bh::MAXS;
}
inline bool bh_lse64_ok(const BwdArgs& a) { return !a.probs && a.D == bh::p64::DK && a.S >= 1 && a.S <= bh::MAXS; }

inline hipError_t launch_bh64(const BwdArgs& a, hipStream_t s) {
    const int64_t grid = (int64_t)a.B * a.H;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    const int mode = (a.causal ? 1 : 0) + (a.probs ? 0 : 2);
    static void (*const kerns[4])(BwdArgs) = {bh::bwd_bh64_kernel<false, false>, bh::bwd_bh64_kernel<true, false>,
                                              bh::bwd_bh64_kernel<false, true>, bh::bwd_bh64_kernel<true, true>};
    static std::atomic<unsigned long long> attr_set[4] = {{0}, {0}, {0}, {0}};
    hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(kerns[mode]), bh::p64::kLdsBytes, attr_set[mode]);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kerns[mode], dim3((unsigned)grid), dim3(bh::NW * 64), bh::p64::kLdsBytes, s, a);
    return hipGetLastError();
}

}  // namespace bwd
}  // namespace hipgpt
