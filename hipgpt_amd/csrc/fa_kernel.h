// fa_kernel.h -- the MFMA flash-attention forward kernel body, shared by the
// fp32 (fa_f32.hip) and bf16 (fa_bf16.hip) instantiations through a traits
// type that supplies the operand layouts and the two matrix products.
//
// Work decomposition (one workgroup = NQS x NKS waves):
//   * The workgroup owns NQS*32 consecutive queries of one (batch, head).
//     Wave (qs, ks) owns the 32 queries of sub-block qs and every NKS-th
//     key tile starting at tile ks, so a long causal row is split over NKS
//     waves (balance) and the CU holds NKS times more waves (latency hiding).
//   * One stage = NKS key tiles of 32 rows, staged global -> registers ->
//     LDS (K row-major, V transposed), double buffered, one barrier per
//     stage; the next stage's global loads are in flight during compute.
//   * Per tile: S^T = K Q^T (32x32 MFMA accumulator, layout in fa_common.h),
//     mask, online softmax in the log2 domain, O^T += V^T P^T with P taken
//     straight from the accumulator registers.
//   * The NKS partial states (m, l, O) of a query sub-block are merged in
//     LDS at the end (log-sum-exp), or, when probs are written, the row
//     max/sum are merged after sweep 1 and the already normalised partial O
//     are summed after sweep 2.
//   * Causal: tiles above a wave's diagonal are skipped (wave-uniform), only
//     diagonal tiles are masked, query blocks are launched longest-first.
#pragma once

#include <type_traits>
#include <utility>

#include "common.h"
#include "fa_common.h"

namespace hipgpt {
namespace fa {

// Start stagger of short causal grids (see FaKernel::run): 35 ticks of the
// 100 MHz s_memrealtime counter = 350 ns per launch rank, for grids of at
// most 4 query blocks per (batch, head) that are resident at once and fill
// at least half of the device's workgroup slots (c1: 16.1 -> 15.8 us against 200 ns;
// measured over 100 .. 800 ns per rank; re-measured on cache-rotated inputs
// at 250 .. 550 ns: within 0.1 us rotated, 350 ns best hot).
constexpr unsigned long long kStaggerTicks = 35;
// The same for grids that write probs: 1 us per rank without a causal mask
// (c1 drop-in 31.3 -> 29.9 us), 700 ns with one (c1 with probs 25.0 ->
// 24.7 us); measured over 0.4 .. 1.6 us per rank.
constexpr unsigned long long kStaggerTicksProbs = 100;
constexpr unsigned long long kStaggerTicksProbsCausal = 70;
// Probs tiles of the score-resident sweep, and of the causal probs sweeps at
// padded head dims >= kTransOwnMinDP (one workgroup per CU, LDS to spare),
// are stored through a per-wave LDS transpose as whole 128-byte rows,
// non-temporally, instead of straight from the accumulator layout (32 bytes
// per row per instruction).  Measured (cache-rotated / hot, us): c1 with probs
// 31.2 / 24.5 -> 28.6 / 24.6, the c1 drop-in 34.9 / 29.6 -> 33.1 / 30.0,
// B = 128 drop-in 138.7 / 124.2 -> 124.7 / 111.2; plain (not non-temporal)
// whole-row stores gained less rotated and lost hot.  The spilled scores of
// those causal sweeps leave the same way.
constexpr int kTransOwnMinDP = 128;
// O stores of the streaming kernel go through a per-wave LDS transpose as
// whole rows of the head, non-temporally: c1 17.85 -> 16.84 us (cache-rotated;
// hot 15.77 -> 14.95), the c1 drop-in 33.2 -> 31.4 us; the transpose with
// plain stores measured level, and non-temporal stores of the accumulator
// layout's 32-byte row pieces were slower (c1 17.6 us).
// Start stagger only for grids of at most this many query blocks per (b, h).
constexpr int kStaggerMaxBlocks = 4;

// SRT > 0 (probs only): when a wave's key tiles span at most SRT stages, the
// max/sum sweep keeps every score tile in registers and the probs sweep reads
// them back instead of recomputing Q K^T (it stages V only).
// SRT < 0 (probs only, rows longer than that): the max/sum sweep stores each
// masked score tile into the probs buffer, where the probs sweep reads it back
// and overwrites it with P -- two products instead of three (no second Q K^T,
// no K staging) for one more write and read of the probs rows.  With the
// accumulator-layout stores each lane reads back only what it wrote, in the
// same sweep order.  With the per-wave LDS transpose (TRANS_OWN: causal, padded
// head dim >= 128) a tile's scores leave as whole rows, so lanes write other
// lanes' rows and the read-back is cross-lane: it is correct only because every
// sweep iteration ends with a workgroup barrier (and one precedes the first
// read-back prefetch), which orders each global store before the loads of the
// other lanes.  A change that removes those barriers breaks the spill.
template <class TR, int NQS, int NKS, bool CAUSAL, bool PROBS, bool VEC, int SRT = 0>
struct FaKernel {
    static constexpr int DP = TR::DP;
    static constexpr int NW = NQS * NKS;
    static constexpr int NT = NW * 64;
    static constexpr int NDB = DP / 32;
    static constexpr bool SPILL = SRT < 0;
    using E = typename TR::elem;

    // LDS: two stage buffers of NKS (K tile + V^T tile); the end-of-kernel
    // merge reuses the same memory.
    static constexpr int STAGE_ELEMS = NKS * (TR::KTILE + TR::VTILE);
    static constexpr int STAGE_BYTES = STAGE_ELEMS * (int)sizeof(E);
    static constexpr int MERGE_BYTES = NKS > 1 ? NW * 64 * (16 * NDB + 2) * 4 : 0;  // key-split merge only
    static constexpr int BASE_BYTES = (2 * STAGE_BYTES > MERGE_BYTES) ? 2 * STAGE_BYTES : MERGE_BYTES;
    // Probs stores through a per-wave LDS transpose (see store_t): the score-
    // resident sweep borrows the idle K half of the stage buffers; the causal
    // probs sweeps at padded D >= kTransOwnMinDP (one workgroup
    // per CU, LDS to spare) get a region of their own after BASE_BYTES, for
    // the spilled scores and the probs alike (B4 H16 S2048 D128 with probs
    // 880 -> 867 us).  Unmasked there, the transpose measured slower (the
    // drop-in 1391 -> 1465 us).
    static constexpr bool TRANS_RES = SRT > 0 && sizeof(E) == 4 && TR::KTILE >= QW * 36 && NW <= 2 * NKS;
    static constexpr bool TRANS_OWN = PROBS && CAUSAL && SRT <= 0 && sizeof(E) == 4 && DP >= kTransOwnMinDP;
    static constexpr int LDS_BYTES = BASE_BYTES + (TRANS_OWN ? NW * QW * 36 * 4 : 0);
    // Without probs, the first stage stages K alone: the first Q K^T waits for
    // the K rows only, V of that stage is requested once K has landed and is
    // stored while the first tile's softmax runs (one more workgroup barrier).
    // Cache-rotated: c1 (fp32, D = 32) 16.86 -> 16.62 us, c3-bf16 31.14 ->
    // 30.38 us; fp32 D = 64 (c3) 128.3 -> 128.8 us and D = 128 (c4) level, so
    // those keep the joint first stage.
    static constexpr bool K_FIRST = !PROBS && (sizeof(E) == 2 || DP == 32);
    // Online-softmax sweeps with 16-byte loads test the running max through
    // the exponentials' sum (kLazySum) after each wave's first tile.
    // Cache-rotated, two interleaved repetitions: c1 16.63 -> 16.56 us, c3
    // 127.9 -> 127.4, c3-bf16 29.56 -> 29.24, c4 580.2 -> 576.7; without a
    // causal mask at the c4 shape 1077 -> 1066, at c3-bf16's 47.4 -> 47.0,
    // the c1 and c3 shapes level; results unchanged bit for bit.  The
    // guarded-load instances (padded head dims) spill registers with it
    // (25 at D = 128) and keep the max test.
    static constexpr bool SUM_CHECK = VEC;
    // Causal grids larger than the device holds at once start their last
    // launch ranks (the shortest query blocks) as slots free, well into the
    // call, on Q rows nobody has read: each workgroup of rank r reads the Q
    // rows of rank r + pf_ranks (same (b, h), same XCD) once during its
    // second stage, one 4-byte load per 64 bytes of row, so those rows come
    // from the caches when that workgroup starts.  Cache-rotated, two
    // interleaved repetitions: c3-bf16 29.7 -> 29.1 us, bf16 B16 H12 S1024
    // 50.0 -> 47.2, c3 127.0 -> 126.5, fp32 B16 H12 S1024 228.6 -> 226.4;
    // fp32 D = 32 (B32 H8 S1024 155.8 -> 157.0) and D = 128 (c4 577 -> 579)
    // measured level or slower and go without.
    static constexpr bool PF_LATE = CAUSAL && !PROBS && (sizeof(E) == 2 || DP == 64);
    // Score-resident sweeps over at most two stages at D = 32 (the small
    // problems' 1 x 4 workgroups: HipGPT's generation call): K and V of both
    // stages are requested at once into the two stage buffers, so neither
    // sweep waits on a load after the first (each stage's loads were
    // otherwise requested one stage, ~0.5 us of compute, before use).
    static constexpr bool LOAD_ALL = SRT == 2 && DP == 32;
    // O stores through LDS, one 32-dim block at a time (whole 128-byte row
    // segments per lane group), with a 32 x 36 scratch per storing wave
    // (ks == 0) inside the LDS already allocated: past the merge area when it
    // fits there, else over it after a barrier.  Only with 16-byte rows of the
    // full padded head (VEC, D = DP).
    static constexpr int O_SCR = NQS * QW * 36 * 4;
    static constexpr bool O_TRANS = VEC && O_SCR <= BASE_BYTES;
    static constexpr bool O_TRANS_PAST = MERGE_BYTES + O_SCR <= BASE_BYTES;

    // Global -> register staging of one stage (K and V), 16-byte chunks.
    static constexpr int EPC = 16 / (int)sizeof(E);      // elements per chunk
    static constexpr int CPR = DP / EPC;                  // chunks per row
    static constexpr int CPS = NKS * BK * CPR;            // chunks per stage (K or V)
    static constexpr int PER = (CPS + NT - 1) / NT;

    // 16-byte loads go through buffer resources whose range is the (b, h)
    // slice's valid K / V rows: rows past Sk read as zero without a
    // predicate, and each load costs one 32-bit offset add.  (Non-VEC
    // problems -- D below the padded dim or unaligned strides -- use plain
    // guarded loads.)
    struct Stager {
        typename TR::chunk kr[PER], vr[PER];  // one stage of K and V chunks
        int koff[PER], voff[PER];  // byte offsets of this thread's chunks from the stage's first row
        __amdgpu_buffer_rsrc_t krs, vrs;
        int kstage, vstage;        // bytes per stage of NKS*BK rows
        const E *Kp, *Vp;
        int64_t kts, vts;
        int Sk, D;

        __device__ __forceinline__ void init(const E* Kp_, const E* Vp_, int64_t kts_, int64_t vts_, int Sk_, int D_,
                                             int tid) {
            Kp = Kp_;
            Vp = Vp_;
            kts = kts_;
            vts = vts_;
            Sk = Sk_;
            D = D_;
            if (VEC) {
                constexpr int ES = (int)sizeof(E);
                krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<E*>(Kp), 0,
                                                        (int)(((int64_t)(Sk - 1) * kts + D) * ES), kBufferFlags);
                vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<E*>(Vp), 0,
                                                        (int)(((int64_t)(Sk - 1) * vts + D) * ES), kBufferFlags);
                kstage = (int)(NKS * BK * kts * ES);
                vstage = (int)(NKS * BK * vts * ES);
#pragma unroll
                for (int i = 0; i < PER; ++i) {
                    const int f = tid + i * NT;
                    const int row = f / CPR;
                    const int cc = f % CPR;
                    koff[i] = (int)((row * kts + cc * EPC) * ES);
                    voff[i] = (int)((row * vts + cc * EPC) * ES);
                }
            }
        }

        template <bool WV = true, bool WK = true>
        __device__ __forceinline__ void load(int stage, int tid) {
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = tid + i * NT;
                if (VEC) {
                    if (CPS % NT == 0 || f < CPS) {
                        if (WK)
                            kr[i] = TR::from_u32x4(__builtin_amdgcn_raw_buffer_load_b128(krs, koff[i] + stage * kstage, 0, 0));
                        if (WV)
                            vr[i] = TR::from_u32x4(__builtin_amdgcn_raw_buffer_load_b128(vrs, voff[i] + stage * vstage, 0, 0));
                    }
                } else {
                    const int row = f / CPR;  // 0 .. NKS*BK-1
                    const int cc = f % CPR;
                    const int key = stage * NKS * BK + row;
                    const bool ok = (CPS % NT == 0 || f < CPS) && key < Sk;
                    if (WK) kr[i] = TR::template load_chunk<false>(Kp, (int64_t)key * kts, cc, D, ok);
                    if (WV) vr[i] = TR::template load_chunk<false>(Vp, (int64_t)key * vts, cc, D, ok);
                }
            }
        }
        template <bool WV = true, bool WK = true>
        __device__ __forceinline__ void store(E* stage, int tid) const {
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = tid + i * NT;
                if (CPS % NT != 0 && f >= CPS) break;
                const int row = f / CPR;
                const int cc = f % CPR;
                const int kt = row / BK;  // tile within the stage
                const int r = row % BK;
                E* Kt = stage + kt * TR::KTILE;
                E* Vt = stage + NKS * TR::KTILE + kt * TR::VTILE;
                if (WK) TR::store_k_chunk(Kt, r, cc, kr[i]);
                if (WV) TR::store_vt_chunk(Vt, r, cc, vr[i]);
            }
        }
    };

    __device__ __forceinline__ static void run(const AttnArgs& a, unsigned char* lds_raw, int* simd_slots) {
        E* const lds = reinterpret_cast<E*>(lds_raw);
        const int tid = threadIdx.x;
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int c = lane & 31;
        const int hf = lane >> 5;
        const int BH = a.B * a.H;
        const int bh = blockIdx.x % BH;
        const int rank = blockIdx.x / BH;
        // query block of a launch rank: longest rows first, except that
        // rank short_rank - 1 (when set) takes the shortest block
        auto qb_of = [&](int r) {
            if (!CAUSAL) return r;
            const int sr = a.short_rank - 1;
            if (r == sr) return 0;
            return a.n_qblk - 1 - (sr >= 0 && r > sr ? r - 1 : r);
        };
        const int qb = qb_of(rank);
        // Rotating the (sub-block, split) roles with the launch rank over the
        // waves ranked by SIMD gives each SIMD a different role in each of
        // the co-resident workgroups, evening out causal work.  Roles are
        // wave-uniform (scalar registers), so tile indexing stays scalar.
        const int sr = simd_rank<NW>(simd_slots, wave, lane);
        int role = (sr + rank) % NW;
        if (CAUSAL && NW == 8) {
            // Two waves per SIMD: the second takes the mirror (NQS-1-qs,
            // NKS-1-ks) of the first's role, so in the diagonal stages, where
            // sub-block qs stops after its own diagonal tile, the waves still
            // busy sit on different SIMDs (c3 128.4 -> 127.1 us, c4 604 -> 586).
            const int b = ((sr >> 1) + rank) % 4;
            const int qb0 = b / NKS, kb0 = b % NKS;
            role = (sr & 1) ? (NQS - 1 - qb0) * NKS + (NKS - 1 - kb0) : qb0 * NKS + kb0;
        }
        const int qs = role / NKS;
        const int ks = role % NKS;
        const int b = bh / a.H;
        const int h = bh % a.H;

        const int q0 = qb * (NQS * QW);
        const int qw0 = q0 + qs * QW;
        const int qi = qw0 + c;
        const int Sq = a.Sq, Sk = a.Sk, off = a.causal_off;

        const E* Qp = static_cast<const E*>(a.q) + b * a.q_bs + h * a.q_hs;
        const E* Kp = static_cast<const E*>(a.k) + b * a.k_bs + h * a.k_hs;
        const E* Vp = static_cast<const E*>(a.v) + b * a.v_bs + h * a.v_hs;

        // Short causal problems (a few query blocks per (batch, head), the
        // grid filling the device's resident slots) start with every workgroup loading its
        // first stage at the same moment, and the first tile computes only
        // when that burst has drained.  Launch rank r waits r * 350 ns first,
        // so the longest query blocks (rank 0) get their operands earliest
        // and compute while the shorter ones load (c1: 16.4 -> 15.9 us).
        // Writing probs, the ranks are spread further apart, so one rank's
        // probs stores (the second sweep, HBM-bound) overlap the next rank's
        // score sweep (MFMA-bound) instead of every workgroup storing at once.
        // Only the workgroups the device starts together (block ids below
        // stagger_slots, set by the launcher when the whole grid is resident at
        // once and fills at least half of the slots) are delayed: a small grid
        // has no burst to spread, and a grid larger than the device starts its
        // later workgroups as slots free up (B = 128 measured the same with and
        // without the stagger).
        if ((CAUSAL || PROBS) && rank > 0 && (int)blockIdx.x < a.stagger_slots) {
            const unsigned long long ticks = PROBS ? (CAUSAL ? kStaggerTicksProbsCausal : kStaggerTicksProbs) : kStaggerTicks;
            const unsigned long long t_end = __builtin_amdgcn_s_memrealtime() + (unsigned long long)rank * ticks;
            for (int i = 0; i < 1024 && __builtin_amdgcn_s_memrealtime() < t_end; ++i) __builtin_amdgcn_s_sleep(2);
        }
        const TileRange tr = tile_range<CAUSAL>(q0, qw0, NQS * QW, Sq, Sk, off);
        const int nstages = (tr.ntiles + NKS - 1) / NKS;
        const int wtiles = tr.wtiles;

        const uint32_t* pf_ptr = nullptr;  // PF_LATE: this thread's 4 bytes of a later block's Q rows
        if (PF_LATE && a.pf_ranks > 0 && rank + a.pf_ranks < a.n_qblk) {
            const int pqb = qb_of(rank + a.pf_ranks);
            constexpr int LPR = (DP * (int)sizeof(E) + 63) / 64;  // 64-byte pieces per row
            const int row = pqb * NQS * QW + tid / LPR, piece = tid % LPR;
            const int col = piece * (64 / (int)sizeof(E));  // inside the row's D elements only
            if (tid < NQS * QW * LPR && row < Sq && col < a.D)
                pf_ptr = reinterpret_cast<const uint32_t*>(Qp + (int64_t)row * a.q_ts + col);
        }
        uint32_t pfv = 0;
        // the load's result is kept (an empty asm reads it) one stage later
        auto pf_issue = [&](int i) {
            if (PF_LATE && i == 1 && pf_ptr) pfv = *pf_ptr;
        };
        auto pf_keep = [&](int i) {
            if (PF_LATE && i == 1) asm volatile("" ::"v"(pfv));
        };

        typename TR::QReg qreg;
        TR::template load_q<VEC>(qreg, Qp + (int64_t)qi * a.q_ts, hf, qi < Sq, a.D, a.qscale);
        const float sc = TR::score_scale(a.qscale);

        floatx16 o[NDB];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[db][r] = 0.f;

        float m_run = kMaxInit;
        float l_run = 0.f;

        auto tile_scores = [&](const E* stage, int t) -> floatx16 {
            floatx16 s = TR::qk(stage + (t % NKS) * TR::KTILE, qreg, c, hf);
            if (tr.edge(t, Sk, CAUSAL, qw0, off)) mask_tile<CAUSAL>(s, t * BK, hf, qi, Sk, off);
            return s;
        };
        auto vt_of = [&](const E* stage, int t) -> const E* {
            return stage + NKS * TR::KTILE + (t % NKS) * TR::VTILE;
        };

        Stager st;
        st.init(Kp, Vp, a.k_ts, a.v_ts, Sk, a.D, tid);
        // Spilled scores of tile t (register r <-> key tb + acc_key(r, hf)):
        // keys past Sk and rows past Sq were never written and read as -inf.
        auto spilled_scores = [&](const float* prow, int t) -> floatx16 {
            floatx16 s;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int k0 = t * BK + 8 * g + 4 * hf;
                floatx4 v = {kNegInf, kNegInf, kNegInf, kNegInf};
                if (qi < Sq) {
                    if (k0 + 3 < Sk) {
                        v = *reinterpret_cast<const floatx4*>(prow + k0);
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (k0 + j < Sk) v[j] = prow[k0 + j];
                    }
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) s[4 * g + j] = v[j];
            }
            return s;
        };
        // Probs stores through LDS: the wave writes its tile ([query][key], 16
        // keys per lane in the accumulator layout) into a private 32 x 36
        // scratch X and reads it back as 8 whole 128-byte rows per
        // instruction, so every store writes full lines, non-temporally.  X is
        // the wave's own: a memory clobber orders the
        // exchange between its lanes.  prow0: row qw0 of the probs.
        auto store_t = [&](float* X, float* prow0, const floatx16& p, int tb, bool pvec) {
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<floatx4*>(X + c * 36 + 8 * g + 4 * hf) =
                    floatx4{p[4 * g], p[4 * g + 1], p[4 * g + 2], p[4 * g + 3]};
            asm volatile("" ::: "memory");
            const int rr = lane >> 3, cc = 4 * (lane & 7);
            const bool full = pvec && tb + BK <= Sk;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int row = 8 * k + rr;
                const floatx4 v = *reinterpret_cast<const floatx4*>(X + row * 36 + cc);
                if (qw0 + row < Sq) {
                    float* dst = prow0 + (int64_t)row * Sk + tb + cc;
                    if (full) {
                        __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(dst));
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (tb + cc + j < Sk) dst[j] = v[j];
                    }
                }
            }
            asm volatile("" ::: "memory");  // the next tile's writes come after these reads
        };
        float* const Xown = reinterpret_cast<float*>(lds_raw + BASE_BYTES) + wave * QW * 36;

        // ------------------------------------------------------------------
        // One stage of compute on LDS buffer (i & 1).  MODE 0: online softmax
        // + PV.  MODE 1: max/sum only (SPILL: and the scores stored).  MODE 2:
        // probs store + PV with the final (m, l) (SPILL: from the stored scores).
        floatx16 s_next;  // SPILL, probs sweep: the next tile's stored scores, loaded one tile ahead
        auto compute = [&](auto mode_tag, int i, float mlog, float* prow, bool pvec) {
            constexpr int MODE = decltype(mode_tag)::value;
            const E* cur = lds + (i & 1) * STAGE_ELEMS;
            const int t = i * NKS + ks;
            if (t >= wtiles) return;
            floatx16 s;
            if constexpr (SPILL && MODE == 2) {
                s = s_next;
                if (t + NKS < wtiles) s_next = spilled_scores(prow, t + NKS);
            } else {
                s = tile_scores(cur, t);
            }
            typename TR::VReg vreg;
            if (MODE != 1) TR::load_v(vreg, vt_of(cur, t), c, hf);  // in flight during the softmax
            if constexpr (MODE == 0) {
                // lazy rescale: raise the running max only when a row's tile
                // max exceeds it by more than kLazyMax
                auto lazy_exp = [&](floatx16& sv) -> float {
                    const float tmax = tile_max(sv) * sc;
                    if (__any(tmax > m_run + kLazyMax)) {
                        const float m_new = vmax(m_run, tmax);
                        const float alpha = fast_exp2(m_run - m_new);
                        l_run *= alpha;
#pragma unroll
                        for (int db = 0; db < NDB; ++db)
#pragma unroll
                            for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
                        m_run = m_new;
                    }
                    float lsum = kSumInit;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        sv[r] = fast_exp2(fmaf(sv[r], sc, -m_run));
                        lsum += sv[r];
                    }
                    return lsum;
                };
                float ls;
                if (!SUM_CHECK || i == 0) {  // stage 0 holds every wave's first tile
                    ls = lazy_exp(s);
                } else {
                    // the sum test of kLazySum; the max test only when it fails,
                    // with the scores recomputed from the staged K tile
                    ls = kSumInit;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        s[r] = fast_exp2(fmaf(s[r], sc, -m_run));
                        ls += s[r];
                    }
                    if (__any(ls > kLazySum)) {
                        asm volatile("" ::: "memory");  // re-read K: no copy of the first product stays live
                        s = tile_scores(cur, t);
                        ls = lazy_exp(s);
                    }
                }
                l_run += ls;  // this lane half's partial; the halves are summed after the sweep
                TR::pv(vreg, s, o, c, hf);
            } else if constexpr (MODE == 1) {
                if constexpr (SPILL && TRANS_OWN)
                    store_t(Xown, prow - (int64_t)c * Sk, s, t * BK, pvec);
                else if (SPILL && qi < Sq)
                    store_probs_tile(prow, s, t * BK, hf, Sk, pvec);
                const float m_new = vmax(m_run, tile_max(s) * sc);
                float ls = kSumInit;
#pragma unroll
                for (int r = 0; r < 16; ++r) ls += fast_exp2(fmaf(s[r], sc, -m_new));
                l_run = l_run * fast_exp2(m_run - m_new) + halves_sum(ls);
                m_run = m_new;
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) s[r] = fast_exp2(fmaf(s[r], sc, -mlog));
                if constexpr (TRANS_OWN)
                    store_t(Xown, prow - (int64_t)c * Sk, s, t * BK, pvec);
                else if (qi < Sq)
                    store_probs_tile(prow, s, t * BK, hf, Sk, pvec);
                TR::pv(vreg, s, o, c, hf);
            }
        };

        // K_FIRST: stage 0's online-softmax step in two halves around the
        // barrier that publishes V -- the scores and the P factors of tile t
        // with K alone staged, then the P V product.
        auto first_scores = [&]() -> floatx16 {
            floatx16 s;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = 0.f;
            if (ks >= wtiles) return s;
            s = tile_scores(lds, ks);
            const float tmax = tile_max(s) * sc;
            if (__any(tmax > m_run + kLazyMax)) {
                const float m_new = vmax(m_run, tmax);
                const float alpha = fast_exp2(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
                m_run = m_new;
            }
            float ls = kSumInit;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[r] = fast_exp2(fmaf(s[r], sc, -m_run));
                ls += s[r];
            }
            l_run += ls;
            return s;
        };
        auto first_pv = [&](const floatx16& p) {
            if (ks >= wtiles) return;
            typename TR::VReg vreg;
            TR::load_v(vreg, vt_of(lds, ks), c, hf);
            TR::pv(vreg, p, o, c, hf);
        };

        // Stage pipeline: stage i+1 is loaded into registers while stage i is
        // computed, then written to the other LDS buffer.  (Two stages of
        // register prefetch measured no faster at any head dim and cost an
        // occupancy step at D = 32.)
        // With probs, the max/sum sweep (MODE 1) requests the probs sweep's first stage during its last one, so
        // the probs sweep (MODE 2) starts from registers instead of a memory round trip.
        constexpr bool WV2 = true, WK2 = !SPILL;  // what the probs sweep stages
        auto sweep = [&](auto mode_tag, float mlog, float* prow, bool pvec) {
            constexpr int MODE = decltype(mode_tag)::value;
            constexpr bool WV = MODE != 1;              // the max/sum sweep stages no V
            constexpr bool WK = !(SPILL && MODE == 2);  // nor the spilled probs sweep K
            if constexpr (MODE == 0 && K_FIRST) {
                if (nstages > 0) {
                    st.template load<false, true>(0, tid);
                    st.template store<false, true>(lds, tid);
                    st.template load<true, false>(0, tid);
                }
                __syncthreads();
                if (nstages > 0) {
                    const floatx16 p0 = first_scores();
                    st.template store<true, false>(lds, tid);
                    if (nstages > 1) st.template load<true, true>(1, tid);
                    __syncthreads();
                    first_pv(p0);
                    if (nstages > 1) st.template store<true, true>(lds + STAGE_ELEMS, tid);
                    __syncthreads();
                }
                for (int i = 1; i < nstages; ++i) {
                    if (i + 1 < nstages) st.template load<true, true>(i + 1, tid);
                    pf_issue(i);
                    compute(mode_tag, i, mlog, prow, pvec);
                    if (i + 1 < nstages) st.template store<true, true>(lds + ((i + 1) & 1) * STAGE_ELEMS, tid);
                    pf_keep(i);
                    __syncthreads();
                }
                return;
            }
            if (nstages > 0) {
                if (MODE != 2) st.template load<WV, WK>(0, tid);
                st.template store<WV, WK>(lds, tid);
            }
            __syncthreads();
            if constexpr (MODE == 1) {
                // the last stage peeled: it requests the probs sweep's first stage
                for (int i = 0; i + 1 < nstages; ++i) {
                    st.template load<WV, WK>(i + 1, tid);
                    compute(mode_tag, i, mlog, prow, pvec);
                    st.template store<WV, WK>(lds + ((i + 1) & 1) * STAGE_ELEMS, tid);
                    __syncthreads();
                }
                if (nstages > 0) {
                    st.template load<WV2, WK2>(0, tid);
                    compute(mode_tag, nstages - 1, mlog, prow, pvec);
                    __syncthreads();
                }
            } else {
                for (int i = 0; i < nstages; ++i) {
                    if (i + 1 < nstages) st.template load<WV, WK>(i + 1, tid);
                    if (MODE == 0) pf_issue(i);
                    compute(mode_tag, i, mlog, prow, pvec);
                    if (i + 1 < nstages) st.template store<WV, WK>(lds + ((i + 1) & 1) * STAGE_ELEMS, tid);
                    if (MODE == 0) pf_keep(i);
                    __syncthreads();
                }
            }
        };

        // Score-resident probs sweeps (SRT > 0).  Stage I holds tile I*NKS + ks
        // of this wave; sres[I] keeps its masked scores between the sweeps.
        floatx16 sres[SRT > 0 ? SRT : 1];
        // One tile of a score-resident sweep: max/sum (first) or probs + P V (second).
        auto res_tile = [&](auto second_tag, auto ic, const E* cur, float mlog, float* prow, bool pvec) {
            constexpr bool SECOND = decltype(second_tag)::value;
            constexpr int I = decltype(ic)::value;
            const int t = I * NKS + ks;
            if (t >= wtiles) return;
            if (!SECOND) {
                const floatx16 sv = tile_scores(cur, t);
                sres[I] = sv;
                const float m_new = vmax(m_run, tile_max(sv) * sc);
                float ls = kSumInit;
#pragma unroll
                for (int r = 0; r < 16; ++r) ls += fast_exp2(fmaf(sv[r], sc, -m_new));
                l_run = l_run * fast_exp2(m_run - m_new) + halves_sum(ls);
                m_run = m_new;
            } else {
                typename TR::VReg vreg;
                TR::load_v(vreg, vt_of(cur, t), c, hf);
                floatx16 p = sres[I];
#pragma unroll
                for (int r = 0; r < 16; ++r) p[r] = fast_exp2(fmaf(p[r], sc, -mlog));
                if constexpr (TRANS_RES) {
                    float* const X =
                        reinterpret_cast<float*>(lds + (wave / NKS) * STAGE_ELEMS + (wave % NKS) * TR::KTILE);
                    store_t(X, prow - (int64_t)c * Sk, p, t * BK, pvec);
                } else {
                    if (qi < Sq) store_probs_tile(prow, p, t * BK, hf, Sk, pvec);
                }
                TR::pv(vreg, p, o, c, hf);
            }
        };
        auto sweep_res = [&](auto second_tag, float mlog, float* prow, bool pvec) {
            constexpr bool SECOND = decltype(second_tag)::value;  // false: max/sum (K), true: probs + PV (V)
            if constexpr (LOAD_ALL) {
                // both stages requested at once and kept in the two buffers
                if (!SECOND) {
                    Stager st2 = st;
                    if (nstages > 0) st.template load<true, true>(0, tid);
                    if (nstages > 1) st2.template load<true, true>(1, tid);
                    if (nstages > 0) st.template store<true, true>(lds, tid);
                    if (nstages > 1) st2.template store<true, true>(lds + STAGE_ELEMS, tid);
                    __syncthreads();
                }
                static_for(
                    [&](auto ic) {
                        constexpr int I = decltype(ic)::value;
                        if (I < nstages) res_tile(second_tag, ic, lds + I * STAGE_ELEMS, mlog, prow, pvec);
                    },
                    std::make_integer_sequence<int, SRT>{});
                // the merge slots (after the first sweep) and the O merge
                // (after the second) reuse the K half of buffer 0
                __syncthreads();
                return;
            }
            if (nstages > 0) {
                // the probs sweep's first V stage was requested in the max/sum sweep's first stage
                if (!SECOND) st.template load<false, true>(0, tid);
                st.template store<SECOND, !SECOND>(lds, tid);
            }
            __syncthreads();
            static_for(
                [&](auto ic) {
                    constexpr int I = decltype(ic)::value;
                    if (I < nstages) {
                        if (I + 1 < nstages) st.template load<SECOND, !SECOND>(I + 1, tid);
                        if (!SECOND && I == 0) st.template load<true, false>(0, tid);  // V of the probs sweep's first stage
                        res_tile(second_tag, ic, lds + (I & 1) * STAGE_ELEMS, mlog, prow, pvec);
                        if (I + 1 < nstages)
                            st.template store<SECOND, !SECOND>(lds + ((I + 1) & 1) * STAGE_ELEMS, tid);
                        __syncthreads();
                    }
                },
                std::make_integer_sequence<int, (SRT > 0 ? SRT : 1)>{});
        };

        float* const mrg = reinterpret_cast<float*>(lds_raw);  // merge scratch (after a barrier)
        float* const m_slot = mrg;                              // [NW][64]
        float* const l_slot = mrg + NW * 64;                    // [NW][64]
        float* const o_slot = mrg + 2 * NW * 64;                // partial O: [NW][4*NDB][64] float4 (merge
                                                                // without probs) or [NW][16*NDB][64] (with)
        // partial O of wave `w`, register group g of block db, as one 16-byte slot per lane
        auto o_at = [&](int w, int db, int g) {
            return reinterpret_cast<floatx4*>(o_slot) + ((w * NDB + db) * 4 + g) * 64 + lane;
        };

        if (!PROBS) {
            sweep(std::integral_constant<int, 0>{}, 0.f, nullptr, false);
            l_run = halves_sum(l_run);
            if (NKS > 1) {
                // wave ks > 0 publishes (m, l, O); wave ks == 0 merges
                if (ks != 0) {
                    m_slot[role * 64 + lane] = m_run;
                    l_slot[role * 64 + lane] = l_run;
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
#pragma unroll
                        for (int g = 0; g < 4; ++g)
                            *o_at(role, db, g) = floatx4{o[db][4 * g], o[db][4 * g + 1], o[db][4 * g + 2], o[db][4 * g + 3]};
                }
                __syncthreads();
                if (ks == 0) {
                    float M = m_run;
#pragma unroll
                    for (int j = 1; j < NKS; ++j) M = fmaxf(M, m_slot[(role + j) * 64 + lane]);
                    const float w0 = fast_exp2(m_run - M);
                    m_run = M;
                    l_run *= w0;
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
#pragma unroll
                        for (int r = 0; r < 16; ++r) o[db][r] *= w0;
#pragma unroll
                    for (int j = 1; j < NKS; ++j) {
                        const float wj = fast_exp2(m_slot[(role + j) * 64 + lane] - M);
                        l_run = fmaf(l_slot[(role + j) * 64 + lane], wj, l_run);
#pragma unroll
                        for (int db = 0; db < NDB; ++db)
#pragma unroll
                            for (int g = 0; g < 4; ++g) {
                                const floatx4 v = *o_at(role + j, db, g);
#pragma unroll
                                for (int u = 0; u < 4; ++u) o[db][4 * g + u] = fmaf(v[u], wj, o[db][4 * g + u]);
                            }
                    }
                }
            }
        } else {
            // Causal: the zeros above the diagonal need no data, so they are
            // stored before the sweeps, while the first stage's loads are in
            // flight (c1 with probs 26.5 -> 25.2 us against storing them last).
            if (CAUSAL && qw0 < Sq && ks == 0) {
                const bool pv0 = (Sk & 3) == 0 && (reinterpret_cast<uintptr_t>(a.probs) & 15) == 0;
                zero_probs_tail<(SRT > 0)>(a.probs + (int64_t)bh * Sq * Sk, qw0, Sq, Sk, tr.wtiles * BK, lane, pv0);
            }
            float* probs_bh = a.probs + (int64_t)bh * Sq * Sk;
            const bool pvec = (Sk & 3) == 0 && (reinterpret_cast<uintptr_t>(a.probs) & 15) == 0;
            if constexpr (SRT > 0)
                sweep_res(std::false_type{}, 0.f, nullptr, false);
            else
                sweep(std::integral_constant<int, 1>{}, 0.f, probs_bh + (int64_t)qi * Sk, pvec);
            if (NKS > 1) {
                m_slot[role * 64 + lane] = m_run;
                l_slot[role * 64 + lane] = l_run;
                __syncthreads();
                const int w0 = qs * NKS;
                float M = kMaxInit;
#pragma unroll
                for (int j = 0; j < NKS; ++j) M = fmaxf(M, m_slot[(w0 + j) * 64 + lane]);
                float L = 0.f;
#pragma unroll
                for (int j = 0; j < NKS; ++j) L = fmaf(l_slot[(w0 + j) * 64 + lane], fast_exp2(m_slot[(w0 + j) * 64 + lane] - M), L);
                m_run = M;
                l_run = L;
                __syncthreads();  // the stage buffers overwrite the slots next
            }
            // P = exp2(s' - m) / l = exp2(s' - (m + log2 l)): the normalisation
            // rides in the exponent (no multiply per score)
            const float mlog = m_run + __builtin_amdgcn_logf(fmaxf(l_run, 1e-20f));
            if constexpr (SPILL) {
                if (ks < wtiles) s_next = spilled_scores(probs_bh + (int64_t)qi * Sk, ks);
            }
            if constexpr (SRT > 0)
                sweep_res(std::true_type{}, mlog, probs_bh + (int64_t)qi * Sk, pvec);
            else
                sweep(std::integral_constant<int, 2>{}, mlog, probs_bh + (int64_t)qi * Sk, pvec);
            if (NKS > 1) {
                if (ks != 0) {
                    // (scalar slots here: 16-byte ones spill the D = 64 probs kernel under its 128-register cap)
                    float* const os = o_slot + role * 16 * NDB * 64;
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
#pragma unroll
                        for (int r = 0; r < 16; ++r) os[(db * 16 + r) * 64 + lane] = o[db][r];
                }
                __syncthreads();
                if (ks == 0) {
#pragma unroll
                    for (int j = 1; j < NKS; ++j)
#pragma unroll
                        for (int db = 0; db < NDB; ++db)
#pragma unroll
                            for (int r = 0; r < 16; ++r)
                                o[db][r] += o_slot[((role + j) * 16 * NDB + db * 16 + r) * 64 + lane];
                }
            }
            l_run = 1.0f;
        }

        // ---------------- epilogue: O = O^T / l (wave ks == 0) ----------------
        // Row log-sum-exp (natural log) when asked for (no-probs path only):
        // scores are in log2 units of scale * q.k, l = sum 2^(s - m).
        if (!PROBS && a.lse && ks == 0 && hf == 0 && qi < Sq)
            a.lse[(int64_t)bh * Sq + qi] = (m_run + log2f(l_run)) * kLn2;
        if constexpr (O_TRANS) {
            if constexpr (!O_TRANS_PAST) __syncthreads();  // the merge's reads of the area are done
            if (ks == 0) {
                float* const X = reinterpret_cast<float*>(lds_raw + (O_TRANS_PAST ? MERGE_BYTES : 0)) + qs * QW * 36;
                const float linv = __builtin_amdgcn_rcpf(fmaxf(l_run, 1e-20f));
                const int rr = lane >> 3, cc = 4 * (lane & 7);
                float* const o0 = a.o + b * a.o_bs + h * a.o_hs + (int64_t)qw0 * a.o_ts;
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
#pragma unroll
                    for (int g = 0; g < 4; ++g)
                        *reinterpret_cast<floatx4*>(X + c * 36 + 8 * g + 4 * hf) =
                            floatx4{o[db][4 * g] * linv, o[db][4 * g + 1] * linv, o[db][4 * g + 2] * linv,
                                    o[db][4 * g + 3] * linv};
                    asm volatile("" ::: "memory");  // other lanes' writes (the wave's LDS accesses are in order)
#pragma unroll
                    for (int k = 0; k < QW / 8; ++k) {
                        const int row = 8 * k + rr;
                        const floatx4 v = *reinterpret_cast<const floatx4*>(X + row * 36 + cc);
                        if (qw0 + row < Sq) {
                            float* dst = o0 + (int64_t)row * a.o_ts + db * 32 + cc;
                            __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(dst));
                        }
                    }
                    asm volatile("" ::: "memory");  // the next block's writes come after these reads
                }
            }
        } else if (ks == 0 && qi < Sq) {
            const float linv = __builtin_amdgcn_rcpf(fmaxf(l_run, 1e-20f));
            float* orow = a.o + b * a.o_bs + h * a.o_hs + (int64_t)qi * a.o_ts;
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d0 = db * 32 + 8 * g + 4 * hf;
                    const floatx4 v = {o[db][4 * g] * linv, o[db][4 * g + 1] * linv, o[db][4 * g + 2] * linv,
                                       o[db][4 * g + 3] * linv};
                    if (VEC) {
                        *reinterpret_cast<floatx4*>(orow + d0) = v;
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (d0 + j < a.D) orow[d0 + j] = v[j];
                    }
                }
            }
        }
    }
};

// Minimum waves per SIMD the register allocator must allow (traits may set
// WAVES_PER_EU; 1 = no constraint).  Applied to the 16-byte-load (VEC)
// instances only: the guarded-load instances of padded head dims need a few
// more registers and would spill under it.
template <class TR, class = void>
struct waves_per_eu { static constexpr int value = 1; };
template <class TR>
struct waves_per_eu<TR, std::void_t<decltype(TR::WAVES_PER_EU)>> { static constexpr int value = TR::WAVES_PER_EU; };

template <class TR, int NQS, int NKS, bool CAUSAL, bool PROBS, bool VEC, int SRT = 0>
__global__ __launch_bounds__(NQS* NKS * 64) __attribute__((amdgpu_waves_per_eu(VEC ? waves_per_eu<TR>::value : 1)))
void fa_fwd_kernel(AttnArgs a) {
    using K = FaKernel<TR, NQS, NKS, CAUSAL, PROBS, VEC, SRT>;
    __shared__ __attribute__((aligned(16))) unsigned char lds[K::LDS_BYTES];
    __shared__ int simd_slots[NQS * NKS];
    K::run(a, lds, simd_slots);
}

template <class TR, int NQS, int NKS, bool CAUSAL, bool PROBS, bool VEC, int SRT = 0>
hipError_t launch_fa(const AttnArgs& a, hipStream_t stream) {
    AttnArgs args = a;
    args.n_qblk = (a.Sq + NQS * QW - 1) / (NQS * QW);
    const int64_t grid = (int64_t)args.n_qblk * a.B * a.H;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    auto kern = fa_fwd_kernel<TR, NQS, NKS, CAUSAL, PROBS, VEC, SRT>;
    static ResidentSlots cache;  // workgroups of this instance the device holds at once
    args.stagger_slots = 0;
    if ((CAUSAL || PROBS) && args.n_qblk > 1 && args.n_qblk <= kStaggerMaxBlocks) {
        const int slots = cache.get(reinterpret_cast<const void*>(kern), NQS * NKS * 64, 0);
        // only grids the device holds at once, filling at least half of it
        if (slots > 0 && 2 * grid >= slots && grid <= slots) args.stagger_slots = slots;
    }
    // Causal grids of more than one round of resident workgroups but under
    // two: the last whole launch rank of the first round runs the shortest
    // query block instead of the next longest, so its slots free early and
    // the blocks of the second round start sooner.  Cache-rotated, three
    // interleaved repetitions: c3 127.2 -> 125.5 us, c3-bf16 28.9 -> 28.8
    // (hot 26.8 -> 26.2), c3 with probs level; grids of two whole rounds
    // keep the plain order (c4 575 -> 632 with it).
    args.short_rank = 0;
    if (CAUSAL && args.n_qblk > 2) {
        const int slots = cache.get(reinterpret_cast<const void*>(kern), NQS * NKS * 64, 0);
        const int64_t bh = (int64_t)a.B * a.H;
        const int64_t R = slots > 0 ? slots / bh : 0;  // whole launch ranks in the first round
        if (grid > slots && grid < 2 * (int64_t)slots && R >= 2 && R < args.n_qblk) args.short_rank = (int)R;
    }
    args.pf_ranks = 0;
    if (FaKernel<TR, NQS, NKS, CAUSAL, PROBS, VEC, SRT>::PF_LATE) {
        // the first round holds slots / (B*H) whole launch ranks
        const int slots = cache.get(reinterpret_cast<const void*>(kern), NQS * NKS * 64, 0);
        const int64_t bh = (int64_t)a.B * a.H;
        if (slots > 0 && grid > slots && slots >= bh) args.pf_ranks = (int)(slots / bh);
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(NQS * NKS * 64), 0, stream, args);
    return hipGetLastError();
}

// Probs rows that do not fit the score-resident stages spill their scores to
// the probs buffer between the sweeps (1) or recompute Q K^T (0).  Reading a
// spilled 32x32 tile back costs 4 KB per query sub-block whatever the head
// size; recomputing it costs a staged K tile (32 * D * 4 bytes, shared by the
// workgroup) and 32 * 32 * D MFMA work.  The spill measured faster on fp32
// operands at D = 128 (B4 H16 S2048: 1623 -> 1504 us for the drop-in
// launcher) and slower at D = 64 (B8 H12 S1024: 327 -> 388 us), so it is
// used for fp32 operands with a padded head size of 128 or more.
constexpr int kScoreSpillMinDP = 128;

// Score-resident stages of a traits type (PROBS_RES_STAGES; 0 = the probs
// sweeps recompute Q K^T).
template <class TR, class = void>
struct probs_res_stages { static constexpr int value = 0; };
template <class TR>
struct probs_res_stages<TR, std::void_t<decltype(TR::PROBS_RES_STAGES)>> {
    static constexpr int value = TR::PROBS_RES_STAGES;
};

// Instances of one workgroup shape chosen by the runtime flags.  CAUSAL_INST
// false: the caller launches it without a causal mask only, and no causal
// instance is compiled.
template <class TR, int NQS, int NKS, bool VEC, bool CAUSAL_INST = true>
hipError_t launch_fa_flags(const AttnArgs& a, bool causal, bool probs, hipStream_t s) {
    constexpr int SRT = probs_res_stages<TR>::value;
    constexpr bool kSpill = VEC && sizeof(typename TR::elem) == 4 && TR::DP >= kScoreSpillMinDP;
    if constexpr (!CAUSAL_INST) {
        if (causal) return hipErrorInvalidValue;
    }
    // causal and non-causal instances of one choice of PROBS and SRT
    auto by_mask = [&](auto probs_tag, auto srt_tag) -> hipError_t {
        constexpr bool P = decltype(probs_tag)::value;
        constexpr int R = decltype(srt_tag)::value;
        if constexpr (CAUSAL_INST) {
            if (causal) return launch_fa<TR, NQS, NKS, true, P, VEC, R>(a, s);
        }
        return launch_fa<TR, NQS, NKS, false, P, VEC, R>(a, s);
    };
    using yes = std::true_type;
    using no = std::false_type;
    if constexpr (SRT > 0) {
        // every wave's key tiles fit the resident stages (Sk <= SRT * NKS * 32)
        if (probs && ((a.Sk + BK - 1) / BK + NKS - 1) / NKS <= SRT)
            return by_mask(yes{}, std::integral_constant<int, SRT>{});
    }
    // longer rows: the scores are spilled to the probs buffer between the
    // sweeps (16-byte aligned probs rows)
    if constexpr (kSpill) {
        if (probs && (a.Sk & 3) == 0 && (reinterpret_cast<uintptr_t>(a.probs) & 15) == 0)
            return by_mask(yes{}, std::integral_constant<int, -1>{});
    }
    return probs ? by_mask(yes{}, std::integral_constant<int, 0>{}) : by_mask(no{}, std::integral_constant<int, 0>{});
}

// Workgroups of one shape's plain instance (no probs) the device holds at
// once, cached per device; 0 if the occupancy query fails.
template <class TR, int NQS, int NKS, bool CAUSAL, bool VEC>
int fa_resident_slots() {
    static ResidentSlots cache;
    return cache.get(reinterpret_cast<const void*>(fa_fwd_kernel<TR, NQS, NKS, CAUSAL, false, VEC, 0>), NQS * NKS * 64,
                     0);
}

}  // namespace fa
}  // namespace hipgpt
