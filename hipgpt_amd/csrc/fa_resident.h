// fa_resident.h -- attention forward with the whole K/V of a (batch, head)
// resident in LDS, for short sequences (HipGPT's default S = 256).
//
// At S = 256 the streaming kernel (fa_kernel.h) spends a large share of its
// time in the prologue (every workgroup loads Q and its first stage at once)
// and in per-stage barriers that keep waves with unequal causal work in
// lockstep.  Here one workgroup of NQS = 8 waves owns 256 queries of one
// (b, h) and keeps every K tile (row-major) and V^T tile it needs in LDS:
//   * Production: tile t is split over all threads; each thread keeps L
//     tiles of loads in flight in registers, writes its share of tile t to
//     LDS, and the wave then bumps an LDS arrival counter for t.
//   * Consumption: a wave that needs tile t waits until all NW waves have
//     signalled it (bounded spin), then computes it.  Every wave produces
//     tile t before it waits on tile t, so the wait always ends; there is no
//     workgroup barrier after the first, so waves with little causal work
//     finish early instead of idling in lockstep.
//   * Balance: the waves are ranked by the SIMD the hardware placed them on
//     (simd_rank).  With two waves per SIMD, the waves of SIMD s take query
//     sub-blocks s and 7-s, so every SIMD carries the same causal work.
//   * With probs the second sweep re-reads K/V from LDS (no reload).  With at
//     most 8 tiles (D = 64: the LDS holds no more), each wave keeps its masked
//     score tiles in registers between the sweeps, so the probs sweep runs
//     P V only instead of recomputing Q K^T.
// (A variant with each sub-block's key tiles split over two waves, for
// D = 32, measured slower than the streaming kernel there and was removed.)
// The per-tile math (S^T = K Q^T, mask, online softmax, O^T += V^T P^T) is the
// same as the streaming kernel's, through the same operand traits.
#pragma once

#include <atomic>
#include <type_traits>

#include "common.h"
#include "fa_common.h"

namespace hipgpt {
namespace fa {

// Largest LDS footprint of a resident workgroup's tiles (bytes), and of the
// whole workgroup with the O stores' scratch (the kernel's static LDS, the
// SIMD ranking, sits in the rest of the 160 KB).
constexpr int kResidentLdsMax = 152 * 1024;
constexpr int kResidentLdsLimit = 160 * 1024 - 256;

template <class TR, int NQS, int L, bool CAUSAL, bool PROBS>
struct FaResident {
    static_assert(NQS == 8, "8 sub-blocks, two waves per SIMD");
    static constexpr int NW = NQS;
    static constexpr int DP = TR::DP;
    static constexpr int NT = NW * 64;
    static constexpr int NDB = DP / 32;
    using E = typename TR::elem;
    static constexpr int TILE_ELEMS = TR::KTILE + TR::VTILE;
    static constexpr int EPC = 16 / (int)sizeof(E);
    static constexpr int CPR = DP / EPC;                 // 16-byte chunks per row
    static constexpr int CPT = BK * CPR;                 // chunks per tile, K (same for V)
    static constexpr int PER = (2 * CPT + NT - 1) / NT;  // K+V chunks per thread per tile
    static_assert(CPT % 64 == 0, "a wave's chunks are all K or all V");

    // LDS layout: [0, 256) arrival counters, then the tiles.
    static constexpr int HEAD_BYTES = 256;
    // Score tiles kept in registers between the probs sweeps (0: recomputed).
    // The LDS bounds a wave's tiles: ceil(Sk / 32) <= MAX_TILES.
    static constexpr int MAX_TILES = kResidentLdsMax / (TILE_ELEMS * (int)sizeof(E));
    static constexpr int SRES = (PROBS && MAX_TILES <= 8) ? MAX_TILES : 0;
    // O stores through a per-wave 16 x 36 scratch past the tiles (whole
    // 128-byte row segments, non-temporal): c2 33.9 -> 32.8 us.  Not with
    // probs, where the larger LDS footprint measured slower (c2 with probs
    // 41.3 -> 48.6 us, drop-in 56.1 -> 60.3 us).
    static constexpr bool O_TRANS = !PROBS && sizeof(E) == 4;
    static constexpr int O_TRANS_BYTES = O_TRANS ? NW * 16 * 36 * 4 : 0;

    __device__ __forceinline__ static void run(const AttnArgs& a, unsigned char* lds_raw, int ntiles_max,
                                               int* simd_slots) {
        E* const tiles = reinterpret_cast<E*>(lds_raw + HEAD_BYTES);
        int* const cnt = reinterpret_cast<int*>(lds_raw);  // 64 arrival counters

        const int tid = threadIdx.x;
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int c = lane & 31;
        const int hf = lane >> 5;

        const int BH = a.B * a.H;
        const int bh = blockIdx.x % BH;
        const int rank = blockIdx.x / BH;
        const int qb = CAUSAL ? a.n_qblk - 1 - rank : rank;
        const int b = bh / a.H;
        const int h = bh % a.H;
        // Ranked by SIMD, waves 2j and 2j+1 of the ranking sit on SIMD j when
        // the hardware puts two waves on each SIMD: they take sub-blocks j and
        // NQS-1-j.
        const int rk = simd_rank<NW>(simd_slots, wave, lane);
        const int simd = rk / 2;
        const int sub = (rk & 1) ? NQS - 1 - simd : simd;

        const int q0 = qb * (NQS * QW);
        const int qw0 = q0 + sub * QW;
        const int qi = qw0 + c;
        const int Sq = a.Sq, Sk = a.Sk, off = a.causal_off;

        const E* Qp = static_cast<const E*>(a.q) + b * a.q_bs + h * a.q_hs;
        const E* Kp = static_cast<const E*>(a.k) + b * a.k_bs + h * a.k_hs;
        const E* Vp = static_cast<const E*>(a.v) + b * a.v_bs + h * a.v_hs;

        const TileRange tr = tile_range<CAUSAL>(q0, qw0, NQS * QW, Sq, Sk, off);
        const int T = min(tr.ntiles, ntiles_max);  // host guarantees ntiles <= ntiles_max
        const int wtiles = tr.wtiles;

        if (tid < 64) cnt[tid] = 0;
        __syncthreads();

        // ---- producer state: this thread's chunks of every tile ----
        constexpr int ES = (int)sizeof(E);
        const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<E*>(Kp), 0, (int)(((int64_t)(Sk - 1) * a.k_ts + a.D) * ES), kBufferFlags);
        const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<E*>(Vp), 0, (int)(((int64_t)(Sk - 1) * a.v_ts + a.D) * ES), kBufferFlags);
        const int ktile = (int)(BK * a.k_ts * ES);
        const int vtile = (int)(BK * a.v_ts * ES);
        int goff[PER];  // byte offset within tile 0 (K or V)
        bool isv[PER], act[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + i * NT;
            act[i] = (2 * CPT) % NT == 0 || f < 2 * CPT;
            isv[i] = f >= CPT;
            const int g = isv[i] ? f - CPT : f;
            const int row = g / CPR, cc = g % CPR;
            goff[i] = (int)((row * (isv[i] ? a.v_ts : a.k_ts) + cc * EPC) * ES);
        }
        typename TR::chunk ring[L][PER];
        auto issue = [&](int t, auto slot_tag) {
            constexpr int SL = decltype(slot_tag)::value;
#pragma unroll
            for (int i = 0; i < PER; ++i)
                if (act[i]) {
                    // K or V is wave-uniform (a tile's chunks are a multiple
                    // of 64): said so, the load takes one scalar resource
                    // instead of a per-lane select of two, which the compiler
                    // issues as a loop over the distinct resources.
                    if (__builtin_amdgcn_readfirstlane(isv[i] ? 1 : 0))
                        ring[SL][i] = TR::from_u32x4(__builtin_amdgcn_raw_buffer_load_b128(vrs, goff[i] + t * vtile, 0, 0));
                    else
                        ring[SL][i] = TR::from_u32x4(__builtin_amdgcn_raw_buffer_load_b128(krs, goff[i] + t * ktile, 0, 0));
                }
        };
        auto publish = [&](int t, auto slot_tag) {
            constexpr int SL = decltype(slot_tag)::value;
            E* Kt = tiles + t * TILE_ELEMS;
            E* Vt = Kt + TR::KTILE;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                if (!act[i]) continue;
                const int f = tid + i * NT;
                const int g = isv[i] ? f - CPT : f;
                const int row = g / CPR, cc = g % CPR;
                if (isv[i])
                    TR::store_vt_chunk(Vt, row, cc, ring[SL][i]);
                else
                    TR::store_k_chunk(Kt, row, cc, ring[SL][i]);
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
            if (lane == 0) __hip_atomic_fetch_add(&cnt[t], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        };
        auto wait_tile = [&](int t) {
            // Bounded: every wave signals every tile before waiting on it.  An
            // expiry is counted (note_wait_expired) for the host to see.
            for (int spin = 0; spin < (1 << 22); ++spin) {
                if (__hip_atomic_load(&cnt[t], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= NW) return;
                __builtin_amdgcn_s_sleep(1);
            }
            if (lane == 0) note_wait_expired();
        };

        // ---- consumer state ----
        typename TR::QReg qreg;
        TR::template load_q<true>(qreg, Qp + (int64_t)qi * a.q_ts, hf, qi < Sq, a.D, a.qscale);
        const float sc = TR::score_scale(a.qscale);
        floatx16 o[NDB];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
        float m_run = kMaxInit, l_run = 0.f;

        auto scores = [&](int t) -> floatx16 {
            floatx16 s = TR::qk(tiles + t * TILE_ELEMS, qreg, c, hf);
            if (tr.edge(t, Sk, CAUSAL, qw0, off)) mask_tile<CAUSAL>(s, t * BK, hf, qi, Sk, off);
            return s;
        };
        auto online = [&](int t) {
            floatx16 s = scores(t);
            typename TR::VReg vreg;
            TR::load_v(vreg, tiles + t * TILE_ELEMS + TR::KTILE, c, hf);
            // lazy rescale (kLazyMax): raise the running max only when a row's
            // tile max exceeds it by more than the threshold
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
            l_run += ls;  // this lane half's partial; the halves are summed after the loop
            TR::pv(vreg, s, o, c, hf);
        };
        auto stats = [&](int t) {
            const floatx16 s = scores(t);
            const float m_new = vmax(m_run, tile_max(s) * sc);
            float ls = kSumInit;
#pragma unroll
            for (int r = 0; r < 16; ++r) ls += fast_exp2(fmaf(s[r], sc, -m_new));
            l_run = l_run * fast_exp2(m_run - m_new) + halves_sum(ls);
            m_run = m_new;
            return s;
        };
        floatx16 sres[SRES > 0 ? SRES : 1];  // masked scores of tile t (SRES > 0)

        // ---- produce every tile, consume the ones this wave needs ----
        // Production runs L tiles ahead of consumption: tiles 0..L-1 are
        // published before any compute, then tile t+L is published (and
        // t+2L requested) before tile t is computed.  Slot of tile t: t % L
        // (compile-time: the loops are unrolled L times).
        static_assert(L == 2 || L == 4, "ring depth");
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using S2 = std::integral_constant<int, (L == 4 ? 2 : 0)>;
        using S3 = std::integral_constant<int, (L == 4 ? 3 : 1)>;
        auto ahead = [&](int t, auto slot_tag) {  // initial run-ahead for tile t < L
            if (t < T) {
                publish(t, slot_tag);
                if (t + L < T) issue(t + L, slot_tag);
            }
        };
        auto step = [&](int t, auto slot_tag, auto consume) {
            if (t >= T) return;
            if (t + L < T) {
                publish(t + L, slot_tag);
                if (t + 2 * L < T) issue(t + 2 * L, slot_tag);
            }
            if (t < wtiles) {
                wait_tile(t);
                consume(t);
            }
        };
        auto consume = [&](int t) {
            if (PROBS)
                stats(t);
            else
                online(t);
        };
        if (0 < T) issue(0, S0{});
        if (1 < T) issue(1, S1{});
        if (L == 4) {
            if (2 < T) issue(2, S2{});
            if (3 < T) issue(3, S3{});
        }
        ahead(0, S0{});
        ahead(1, S1{});
        if (L == 4) {
            ahead(2, S2{});
            ahead(3, S3{});
        }
        if constexpr (SRES > 0) {
            // T <= SRES: every tile index is a compile-time constant
            static_for(
                [&](auto tc) {
                    constexpr int TT = decltype(tc)::value;
                    step(TT, std::integral_constant<int, TT % L>{}, [&](int t) { sres[TT] = stats(t); });
                },
                std::make_integer_sequence<int, (SRES > 0 ? SRES : 1)>{});
        } else {
            for (int t0 = 0; t0 < T; t0 += L) {
                step(t0, S0{}, consume);
                step(t0 + 1, S1{}, consume);
                if (L == 4) {
                    step(t0 + 2, S2{}, consume);
                    step(t0 + 3, S3{}, consume);
                }
            }
        }

        if (!PROBS) l_run = halves_sum(l_run);
        if (PROBS) {
            // sweep 2 from the resident tiles: P = exp(s - m) / l stored once, P V
            // P = exp2(s' - (m + log2 l)): the normalisation rides in the exponent
            const float mlog = m_run + __builtin_amdgcn_logf(fmaxf(l_run, 1e-20f));
            float* probs_bh = a.probs + (int64_t)bh * Sq * Sk;
            float* prow = probs_bh + (int64_t)qi * Sk;
            const bool pvec = (Sk & 3) == 0 && (reinterpret_cast<uintptr_t>(a.probs) & 15) == 0;
            auto probs_tile = [&](int t, floatx16 s) {
                typename TR::VReg vreg;
                TR::load_v(vreg, tiles + t * TILE_ELEMS + TR::KTILE, c, hf);
#pragma unroll
                for (int r = 0; r < 16; ++r) s[r] = fast_exp2(fmaf(s[r], sc, -mlog));
                if (qi < Sq) store_probs_tile(prow, s, t * BK, hf, Sk, pvec);
                TR::pv(vreg, s, o, c, hf);
            };
            if constexpr (SRES > 0) {
                static_for(
                    [&](auto tc) {
                        constexpr int TT = decltype(tc)::value;
                        if (TT < wtiles) probs_tile(TT, sres[TT]);
                    },
                    std::make_integer_sequence<int, (SRES > 0 ? SRES : 1)>{});
            } else {
                for (int t = 0; t < wtiles; ++t) probs_tile(t, scores(t));
            }
            if (CAUSAL && qw0 < Sq) zero_probs_tail(probs_bh, qw0, Sq, Sk, wtiles * BK, lane, pvec);
            l_run = 1.0f;
        }

        if constexpr (O_TRANS) {
            // O through the wave's 16 x 36 scratch past the tiles, one 32-dim
            // block and 16 query rows at a time: whole 128-byte row segments
            // per lane group, non-temporal
            {
                const int body = ntiles_max * TILE_ELEMS * (int)sizeof(E);
                float* const X = reinterpret_cast<float*>(lds_raw + HEAD_BYTES + body) + wave * 16 * 36;
                const float linv = __builtin_amdgcn_rcpf(fmaxf(l_run, 1e-20f));
                float* const o0 = a.o + b * a.o_bs + h * a.o_hs + (int64_t)qw0 * a.o_ts;
                const int rr = lane >> 3, cc = 4 * (lane & 7);
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        if ((c >> 4) == hh)
#pragma unroll
                            for (int g = 0; g < 4; ++g)
                                *reinterpret_cast<floatx4*>(X + (c - 16 * hh) * 36 + 8 * g + 4 * hf) =
                                    floatx4{o[db][4 * g] * linv, o[db][4 * g + 1] * linv, o[db][4 * g + 2] * linv,
                                            o[db][4 * g + 3] * linv};
                        asm volatile("" ::: "memory");  // other lanes' writes (the wave's LDS accesses are in order)
#pragma unroll
                        for (int k = 0; k < 2; ++k) {
                            const int row = 16 * hh + 8 * k + rr;
                            const floatx4 v = *reinterpret_cast<const floatx4*>(X + (8 * k + rr) * 36 + cc);
                            if (qw0 + row < Sq)
                                __builtin_nontemporal_store(
                                    v, reinterpret_cast<floatx4*>(o0 + (int64_t)row * a.o_ts + db * 32 + cc));
                        }
                        asm volatile("" ::: "memory");  // the next pass's writes come after these reads
                    }
            }
        } else if (qi < Sq) {
            const float linv = __builtin_amdgcn_rcpf(fmaxf(l_run, 1e-20f));
            float* orow = a.o + b * a.o_bs + h * a.o_hs + (int64_t)qi * a.o_ts;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    *reinterpret_cast<floatx4*>(orow + db * 32 + 8 * g + 4 * hf) =
                        floatx4{o[db][4 * g] * linv, o[db][4 * g + 1] * linv, o[db][4 * g + 2] * linv,
                                o[db][4 * g + 3] * linv};
        }
    }
};

template <class TR, int NQS, int L, bool CAUSAL, bool PROBS>
__global__ __launch_bounds__(NQS * 64) void fa_resident_kernel(AttnArgs a, int ntiles_max) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_dyn[];
    __shared__ int simd_slots[NQS];
    FaResident<TR, NQS, L, CAUSAL, PROBS>::run(a, lds_dyn, ntiles_max, simd_slots);
}

// Dynamic-LDS bytes for a resident launch over all ceil(Sk / 32) key tiles
// (the last query block of a causal problem sees every key), or 0 when the
// problem does not fit one workgroup's LDS.
template <class TR, int NQS>
inline size_t resident_lds_bytes(const AttnArgs& a) {
    using R = FaResident<TR, NQS, 4, false, false>;
    const int64_t tiles = ((int64_t)a.Sk + BK - 1) / BK;
    const int64_t body = tiles * R::TILE_ELEMS * (int64_t)sizeof(typename TR::elem);
    using RP = FaResident<TR, NQS, 4, false, true>;
    const int64_t bytes = R::HEAD_BYTES + body + (a.probs ? RP::O_TRANS_BYTES : R::O_TRANS_BYTES);
    return (tiles <= 64 && R::HEAD_BYTES + body <= kResidentLdsMax && bytes <= kResidentLdsLimit) ? (size_t)bytes : 0;
}

template <class TR, int NQS, int L, bool CAUSAL, bool PROBS>
hipError_t launch_resident_one(const AttnArgs& args, int ntiles, size_t lds, int64_t grid, hipStream_t stream) {
    auto kern = fa_resident_kernel<TR, NQS, L, CAUSAL, PROBS>;
    // The dynamic-LDS limit is a per-device function attribute: raise it once
    // per device (bit d of attr_set) and instantiation.  Concurrent first calls
    // may both set it, which is harmless.
    static std::atomic<unsigned long long> attr_set{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const unsigned long long bit = (dev >= 0 && dev < 64) ? 1ull << dev : 0ull;
    if (!bit || !(attr_set.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                kResidentLdsLimit);
        if (e != hipSuccess) return e;
        attr_set.fetch_or(bit, std::memory_order_release);
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(NQS * 64), lds, stream, args, ntiles);
    return hipGetLastError();
}

template <class TR, int NQS, int L>
hipError_t launch_resident(const AttnArgs& a, bool causal, hipStream_t stream) {
    const size_t lds = resident_lds_bytes<TR, NQS>(a);
    if (lds == 0) return hipErrorInvalidConfiguration;
    const int ntiles = (a.Sk + BK - 1) / BK;
    AttnArgs args = a;
    args.n_qblk = (a.Sq + NQS * QW - 1) / (NQS * QW);
    const int64_t grid = (int64_t)args.n_qblk * a.B * a.H;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    const bool probs = a.probs != nullptr;
    if (causal)
        return probs ? launch_resident_one<TR, NQS, L, true, true>(args, ntiles, lds, grid, stream)
                     : launch_resident_one<TR, NQS, L, true, false>(args, ntiles, lds, grid, stream);
    return probs ? launch_resident_one<TR, NQS, L, false, true>(args, ntiles, lds, grid, stream)
                 : launch_resident_one<TR, NQS, L, false, false>(args, ntiles, lds, grid, stream);
}

}  // namespace fa
}  // namespace hipgpt
