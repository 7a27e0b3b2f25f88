// fa_common.h -- pieces shared by the fp32 and bf16 MFMA attention kernels.
//
// Both kernels compute the score tile transposed, S^T = K Q^T, with a
// 32x32 MFMA whose accumulator gives lane l (c = l & 31, h = l >> 5) query
// column c and the 16 key rows acc_key(r, h), r = 0..15.  A query's row
// statistics are therefore an in-lane reduction over 16 registers plus one
// exchange between the two wave halves (v_permlane32_swap), and the
// exponentiated tile is directly the P^T operand of O^T = V^T P^T.
#pragma once

#include <type_traits>
#include <utility>

#include "common.h"

namespace hipgpt {
namespace fa {

constexpr int BK = 32;  // keys per tile
constexpr int QW = 32;  // queries per wave

// Compile-time loop over I = 0 .. N-1 (each body sees I as a constant).
template <class F, int... Is>
__device__ __forceinline__ void static_for(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}

// Rescale threshold of the online softmax (log2 units): the running max of a
// row is only raised when a tile's max exceeds it by more than this, so the
// O / l rescale is skipped on most tiles; exponentiated scores are then at
// most 2^kLazyMax, far from fp32 overflow, and the final O / l is unchanged.
constexpr float kLazyMax = 8.0f;
// After a row's first tile the running max can also be checked without
// forming the tile's max: exponentiate against the running max and test the
// lane's sum of the 16 exponentials against 2^kLazyMax.  No exponential
// exceeds 2^kLazyMax when the sum does not (all are >= 0), which is exactly
// when the max test keeps the running max; a larger sum sends the tile back
// through the max test (scores recomputed), so the results are the same bit
// for bit and the common tile saves the max reduction (8 v_maximum3, a lane
// exchange, a compare).
constexpr float kLazySum = 256.0f;  // 2^kLazyMax
// Start of a sum of exponentials: -0 is the additive identity (x + -0 == x
// for every x), so the first add folds away; from +0 it stays an instruction.
constexpr float kSumInit = -0.0f;

// SIMD of the calling wave (HW_ID.SIMD_ID, bits [5:4]).
__device__ __forceinline__ int wave_simd() { return (__builtin_amdgcn_s_getreg(4 | (4 << 6) | (1 << 11))) & 3; }

// The hardware places a workgroup's waves on the CU's SIMDs in an order that
// varies between workgroups.  Rank each wave by its SIMD (ties by wave id):
// a bijection onto 0..NW-1 that, with one wave per SIMD, is the SIMD id, so
// that roles rotated by the workgroup's launch rank spread causal work evenly
// over the SIMDs.  One barrier; `slots` is NW ints of LDS.
template <int NW>
__device__ __forceinline__ int simd_rank(int* slots, int wave, int lane) {
    const int me = wave_simd();
    if (lane == 0) slots[wave] = me;
    __syncthreads();
    int rk = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const int s = slots[w];
        rk += (s < me) || (s == me && w < wave);
    }
    return __builtin_amdgcn_readfirstlane(rk);
}

// Key (within the tile) held by accumulator register r of lane half h.
__device__ __forceinline__ int acc_key(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// IEEE-754 maximum (NaN-propagating): maps to v_maximum3_f32 on gfx950 and,
// unlike fmaxf, needs no input canonicalisation.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// max / sum of x over lanes l and l ^ 32 (the two halves hold the same query).
__device__ __forceinline__ float halves_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Row max of a score tile: a strict chain, which the compiler folds into
// eight v_maximum3_f32.
__device__ __forceinline__ float tile_max(const floatx16& s) {
    float m = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) m = vmax(m, s[r]);
    return halves_max(m);
}

// Mask scores of keys >= Sk and, causally, keys > query + off: register r
// of lane half hf holds key tb + acc_key(r, hf), visible iff
// acc_key(r, 0) < min(Sk, qi + off + 1) - tb - 4*hf (one compare per score).
template <bool CAUSAL>
__device__ __forceinline__ void mask_tile(floatx16& s, int tb, int hf, int qi, int Sk, int off) {
    int lim = CAUSAL ? min(Sk, qi + off + 1) : Sk;
    lim -= tb + 4 * hf;
#pragma unroll
    for (int r = 0; r < 16; ++r)
        if (!(8 * (r >> 2) + (r & 3) < lim)) s[r] = kNegInf;
}

// Tile loop bounds for a workgroup of NW waves at query block qb.
struct TileRange {
    int ntiles;  // tiles the workgroup loads
    int wtiles;  // tiles this wave computes (a prefix of the above)
    __device__ __forceinline__ bool edge(int t, int Sk, bool causal, int qw0, int off) const {
        const int tb = t * BK;
        return (tb + BK > Sk) || (causal && tb + BK - 1 > qw0 + off);
    }
};

template <bool CAUSAL>
__device__ __forceinline__ TileRange tile_range(int q0, int qw0, int nq_wg, int Sq, int Sk, int off) {
    TileRange r;
    int kend = Sk, wkend = Sk;
    if (CAUSAL) {
        kend = min(Sk, min(q0 + nq_wg, Sq) + off);
        wkend = min(Sk, min(qw0 + QW, Sq) + off);
    }
    r.ntiles = (kend + BK - 1) / BK;
    r.wtiles = (qw0 < Sq) ? (wkend + BK - 1) / BK : 0;
    return r;
}

// Store a P tile (register r of lane (c, hf) -> probs[qi][tb + acc_key(r, hf)]).
__device__ __forceinline__ void store_probs_tile(float* prow, const floatx16& p, int tb, int hf, int Sk, bool pvec) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int k0 = tb + 8 * g + 4 * hf;
        if (pvec && k0 + 3 < Sk) {
            // Plain (not non-temporal) stores: each row gets 32 bytes per
            // instruction, and L2 merges them into full lines (non-temporal
            // partial-line stores measured 2x slower).
            *reinterpret_cast<floatx4*>(prow + k0) = floatx4{p[4 * g], p[4 * g + 1], p[4 * g + 2], p[4 * g + 3]};
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (k0 + j < Sk) prow[k0 + j] = p[4 * g + j];
        }
    }
}

// Causal: zero the probs of this wave's queries for keys >= z0 (whole rows
// per instruction; non-temporal if NT: the score-resident streaming sweep,
// c1 with probs 27.7 -> 26.6 us; the other probs paths measured 1-9% slower
// with it).
template <bool NT = false>
__device__ __forceinline__ void zero_probs_tail(float* probs_bh, int qw0, int Sq, int Sk, int z0, int lane, bool pvec) {
    for (int r = 0; r < QW; ++r) {
        const int q = qw0 + r;
        if (q >= Sq) break;
        float* pr = probs_bh + (int64_t)q * Sk;
        if (pvec) {
            for (int k = z0 + lane * 4; k < Sk; k += 256) {
                if constexpr (NT)
                    __builtin_nontemporal_store(floatx4{0.f, 0.f, 0.f, 0.f}, reinterpret_cast<floatx4*>(pr + k));
                else
                    *reinterpret_cast<floatx4*>(pr + k) = floatx4{0.f, 0.f, 0.f, 0.f};
            }
        } else {
            for (int k = z0 + lane; k < Sk; k += 64) pr[k] = 0.f;
        }
    }
}

}  // namespace fa
}  // namespace hipgpt
