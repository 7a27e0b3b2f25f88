// fa_f32.hip -- exact fp32 attention forward on gfx950 MFMA.
//
// Replaces flash_attention_kernel<32|64> and multihead_attention_kernel_fallback
// (HipGPT src/hip_kernels.cpp:263-325, :329-402) for head dims up to 128
// (D = 16, 48, 96, ... run zero-padded to the next of 32/64/128).  The kernel
// body is fa_kernel.h; this file supplies the fp32 operand traits:
//   * S^T = K Q^T on v_mfma_f32_32x32x2_f32.  Q is held in registers,
//     pre-scaled by scale*log2(e) (so scores are already in the log2
//     domain).  Lane (c, h) takes the contraction indices d = h*DP/2 + s:
//     its K operand is 4 consecutive floats of K row c per ds_read_b128.
//   * O^T = V^T P^T: for accumulator register r the lane needs
//     V[acc_key(r, h)][d]; V is stored transposed in LDS so the four
//     consecutive keys of each register group are one ds_read_b128.
//   * K pitch DP+4 floats and V^T pitch 36 floats keep the 16-lane phases
//     of ds_read_b128 on distinct banks.
//
// MFMA 32x32x2 f32 operand layout (lane l, c = l & 31, h = l >> 5):
//   A[m][k]: lane holds A[c][h]          B[k][n]: lane holds B[h][c]
//   D[m][n]: register r holds D[8*(r/4) + 4*h + (r%4)][c]
#include "common.h"
#include "fa_kernel.h"
#include "fa_resident.h"
#include "kernels.h"

namespace hipgpt {

namespace {

using fa::BK;

template <int DP_, bool VPRE_ = (DP_ <= 32), int SRES_ = (DP_ == 32 ? 4 : 0)>
struct F32Traits {
    static constexpr int DP = DP_;
    using elem = float;
    using chunk = floatx4;
    static constexpr int KSTR = DP + 4;
    static constexpr int VTP = BK + 4;
    static constexpr int KTILE = BK * KSTR;
    static constexpr int VTILE = DP * VTP;

    struct QReg {
        float v[DP / 2];
    };

    template <bool VEC>
    __device__ __forceinline__ static void load_q(QReg& q, const float* qrow, int hf, bool valid, int D,
                                                  float qscale) {
        const float* p = qrow + hf * (DP / 2);
        if (!valid) {
#pragma unroll
            for (int s = 0; s < DP / 2; ++s) q.v[s] = 0.f;
        } else if (VEC) {
#pragma unroll
            for (int s = 0; s < DP / 2; s += 4) {
                const floatx4 t = *reinterpret_cast<const floatx4*>(p + s);
#pragma unroll
                for (int j = 0; j < 4; ++j) q.v[s + j] = t[j] * qscale;
            }
        } else {
#pragma unroll
            for (int s = 0; s < DP / 2; ++s) q.v[s] = (hf * (DP / 2) + s < D) ? p[s] * qscale : 0.f;
        }
    }

    __device__ __forceinline__ static chunk from_u32x4(u32x4 v) { return __builtin_bit_cast(chunk, v); }

    // Q already carries scale*log2(e).
    __device__ __forceinline__ static float score_scale(float) { return 1.0f; }

    template <bool VEC>
    __device__ __forceinline__ static chunk load_chunk(const float* base, int64_t rowoff, int cc, int D, bool ok) {
        if (VEC) return ok ? *reinterpret_cast<const floatx4*>(base + rowoff + cc * 4) : floatx4{0.f, 0.f, 0.f, 0.f};
        chunk r;
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = (ok && cc * 4 + j < D) ? base[rowoff + cc * 4 + j] : 0.f;
        return r;
    }
    __device__ __forceinline__ static void store_k_chunk(float* Kt, int r, int cc, const chunk& v) {
        *reinterpret_cast<floatx4*>(Kt + r * KSTR + cc * 4) = v;
    }
    __device__ __forceinline__ static void store_vt_chunk(float* Vt, int r, int cc, const chunk& v) {
#pragma unroll
        for (int j = 0; j < 4; ++j) Vt[(cc * 4 + j) * VTP + r] = v[j];
    }

    // K operands are read in groups of up to 8 x 16 bytes ahead of the MFMA
    // chain (the whole tile for DP <= 64), so the LDS latency is paid once
    // per group rather than per read.
    static constexpr int KG = DP / 8 < 8 ? DP / 8 : 8;
    __device__ __forceinline__ static floatx16 qk(const float* Kt, const QReg& q, int c, int hf) {
        const float* kr = Kt + c * KSTR + hf * (DP / 2);
        floatx16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
        for (int j0 = 0; j0 < DP / 8; j0 += KG) {
            floatx4 kv[KG];
#pragma unroll
            for (int j = 0; j < KG; ++j) kv[j] = *reinterpret_cast<const floatx4*>(kr + 4 * (j0 + j));
#pragma unroll
            for (int j = 0; j < KG; ++j)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[j][u], q.v[4 * (j0 + j) + u], s, 0, 0, 0);
        }
        return s;
    }

    // V^T operands of a tile: lane (c, hf) of block db needs
    // V[acc_key(t, hf)][db*32 + c], t = 0..15 -- four ds_read_b128 per block.
    // VPRE: read before the softmax (VReg holds them) -- the streaming kernel
    // at DP = 32 and the resident kernel; otherwise each block is read just
    // before use.  That brings the streaming kernel at DP = 64 to 128 VGPRs:
    // with WAVES_PER_EU = 4 two 8-wave workgroups share a CU (c3: 132 -> 128
    // us; prefetching V under the same cap spills).
    static constexpr bool VPRE = VPRE_;
    static constexpr int WAVES_PER_EU = (DP == 64 && !VPRE) ? 4 : 1;
    // With probs, rows of up to SRES stages keep their score tiles in
    // registers between the two sweeps (DP = 32: 4 stages, Sk <= 256 at two
    // key splits).
    static constexpr int PROBS_RES_STAGES = SRES_;
    struct VReg {
        floatx4 v[VPRE ? DP / 32 : 1][4];
        const float* vt;
    };
    __device__ __forceinline__ static void load_block(floatx4 (&dst)[4], const float* Vt, int db, int c, int hf) {
        const float* p = Vt + (db * 32 + c) * VTP + 4 * hf;
#pragma unroll
        for (int g = 0; g < 4; ++g) dst[g] = *reinterpret_cast<const floatx4*>(p + 8 * g);
    }
    __device__ __forceinline__ static void load_v(VReg& vr, const float* Vt, int c, int hf) {
        vr.vt = Vt;
        if (VPRE)
#pragma unroll
            for (int db = 0; db < DP / 32; ++db) load_block(vr.v[VPRE ? db : 0], Vt, db, c, hf);
    }
    __device__ __forceinline__ static void pv(const VReg& vr, const floatx16& p, floatx16* o, int c, int hf) {
#pragma unroll
        for (int db = 0; db < DP / 32; ++db) {
            floatx4 blk[4];
            if (VPRE) {
#pragma unroll
                for (int g = 0; g < 4; ++g) blk[g] = vr.v[VPRE ? db : 0][g];
            } else {
                load_block(blk, vr.vt, db, c, hf);
            }
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(blk[g][u], p[4 * g + u], o[db], 0, 0, 0);
        }
    }
};

// Workgroup shape per padded head dim: NQS query sub-blocks x NKS key splits,
// measured on MI355X with waves ranked by SIMD: D=32 2x2 (c1), D=64 4x2 (c3),
// D=128 8x1 (c4) -- the larger head dims run 2 waves per SIMD, and more query
// sub-blocks per workgroup share each K/V stage.
template <int DP, int NQS, int NKS, bool CAUSAL_INST = true>
hipError_t launch_dp(const AttnArgs& a, bool causal, bool probs, bool vec, hipStream_t s) {
    return vec ? fa::launch_fa_flags<F32Traits<DP>, NQS, NKS, true, CAUSAL_INST>(a, causal, probs, s)
               : fa::launch_fa_flags<F32Traits<DP>, NQS, NKS, false, CAUSAL_INST>(a, causal, probs, s);
}

// D = 64 without a causal mask: where the 4 x 2 grid needs more than one
// round of resident workgroups, 4 x 1 workgroups (the same 128 queries, no
// key split, half the CU each, so twice as many resident).  Cache-rotated:
// B8 H12 S1024 (768 workgroups on 512 4 x 2 slots) 206.5 -> 198.3 us, the
// HipGPT drop-in there 324.9 -> 320.4 us.  Causal grids measured slower with
// 4 x 1 at every size tried (c3 127 -> 140 us, B16 H12 S1024 229 -> 249,
// c3 with probs 226 -> 245, S = 256 31.1 -> 33.0): their longest rows,
// unsplit, set the end.
// D = 32 causal without probs on rows of at most 256 keys (at most four
// query blocks of 64): where the grid exceeds one round of 2 x 1 workgroups
// (64 queries, no key split, 2 waves), those instead of 2 x 2 -- the key
// split's merge and per-workgroup stage then cost more than its shorter
// rows save, the dispatch balancing the many rounds.  Cache-rotated (G
// workgroups against 2048 2 x 1 slots): c1's shape at B = 128 (G 4096)
// 59.6 -> 54.1 us, B = 256 115.7 -> 109.0; level or slower at B = 48 / 64
// (28.0 / 28.0, 32.5 / 32.0), with probs (B = 128: 101.9 -> 137.7), without
// a causal mask (85.5 / 85.6), and on longer rows (S = 512 B32: 48.9 ->
// 51.5, S = 1024 B8 47.5 -> 64.5, B32 154.8 -> 153.0); c1 itself (G 1024)
// 16.7 -> 20.6.
bool dp32_unsplit(const AttnArgs& a, bool causal, bool probs, bool vec) {
    if (!causal || probs || !vec || a.Sq > 256 || a.Sk > 256) return false;
    const int64_t grid = (int64_t)((a.Sq + 63) / 64) * a.B * a.H;
    const int slots = fa::fa_resident_slots<F32Traits<32>, 2, 1, true, true>();
    return slots > 0 && grid > slots;
}

bool dp64_narrow(const AttnArgs& a, bool causal) {
    if (causal) return false;
    const int64_t grid = (int64_t)((a.Sq + 127) / 128) * a.B * a.H;
    const int slots = fa::fa_resident_slots<F32Traits<64>, 4, 2, false, true>();
    return slots > 0 && grid > slots;
}

}  // namespace

hipError_t fa_f32_wait_expired(unsigned int* count, bool clear) { return wait_expired_take(count, clear); }

int fa_f32_padded_dim(int D) {
    if (D <= 32) return 32;
    if (D <= 64) return 64;
    if (D <= 128) return 128;
    return 0;
}

// Probs rows of 193 to 256 keys at DP = 64 (all K/V tiles of a (b, h) fit one
// workgroup's LDS) run the resident kernel: 8 waves = 256 queries per
// workgroup, the scores kept between the sweeps.  Cache-rotated, B*H = 256:
// S = 256 with probs 40.6 (causal) / 55.3 us (drop-in) against 50.7 / 65.0
// for the streaming kernel.  Everything else streams: without probs the
// streaming kernel measured 31.2 against 32.7 us at S = 256 (causal; 44.3
// against 45.4 non-causal), 23.4 against 33.4 at S = 128 and 40.8 against
// 55.8 at S = 192; with probs at S = 128 / 192, 35.6 / 55.6 against 41.9 /
// 68.5 us causal and level / 73.1 against 75.4 non-causal.  At DP = 32 the
// streaming kernel measured faster at every S (17.2 against 17.5 us at c1).
constexpr int kResidentMinSq = 193, kResidentMaxSq = 256;

// Small D <= 32 problems (at most 128 query tiles of 32 rows in all, 128 to
// 256 keys -- HipGPT's generation call, B = 1, H = 8, S = 256, is 64 tiles):
// the 2 x 2 workgroups would put one or two waves on a few dozen SIMDs, so
// each query sub-block is split over 4 waves instead (1 x 4, at most two
// stages of key tiles each, scores kept in registers with probs).  The
// generation call 12.6 -> 9.2 us, B = 1 causal 9.5 -> 7.5 us; from 256 query
// tiles on the two shapes measure the same, and below 128 keys a split would
// hold no tile.  (1 x 8 measured 9.4 us on the generation call, 1 x 2 12.3,
// 2 x 4 12.5.)
constexpr int kSmallNqs = 1, kSmallNks = 4, kSmallMaxQtiles = 128;
// The same split at D = 64 replaces the resident kernel (one 8-wave
// workgroup per (b, h), latency-bound when B*H is far below the CU count)
// up to 512 query tiles: the generation call at E = 512 (B = 1, H = 8,
// S = 256, drop-in) 47.1 -> 12.8 us, B = 8 drop-in 52.0 -> 26.9 us, B = 8
// causal 29.8 -> 20.3 us; at B = 16 (1024 tiles) the causal resident kernel
// is faster (31.0 against 38.7 us).
constexpr int kSmall64MaxQtiles = 512;

hipError_t launch_fa_f32(const AttnArgs& a, bool causal, bool vec, hipStream_t stream) {
    const bool probs = a.probs != nullptr;
    {
        constexpr int NQ = kSmallNqs, NK = kSmallNks, ST = 8 / NK;
        using TS = F32Traits<32, true, ST>;
        const int64_t qtiles = (int64_t)a.B * a.H * ((a.Sq + 31) / 32);
        const bool small = vec && a.Sk >= 128 && a.Sk <= 256 && qtiles <= kSmallMaxQtiles;
        if (small && fa_f32_padded_dim(a.D) == 32) {
            if (probs)
                return causal ? fa::launch_fa<TS, NQ, NK, true, true, true, ST>(a, stream)
                              : fa::launch_fa<TS, NQ, NK, false, true, true, ST>(a, stream);
            return causal ? fa::launch_fa<TS, NQ, NK, true, false, true>(a, stream)
                          : fa::launch_fa<TS, NQ, NK, false, false, true>(a, stream);
        }
        using T6 = F32Traits<64, true, ST>;
        if (vec && a.Sk >= 128 && a.Sk <= 256 && qtiles <= kSmall64MaxQtiles && fa_f32_padded_dim(a.D) == 64) {
            if (probs)
                return causal ? fa::launch_fa<T6, NQ, NK, true, true, true, ST>(a, stream)
                              : fa::launch_fa<T6, NQ, NK, false, true, true, ST>(a, stream);
            return causal ? fa::launch_fa<T6, NQ, NK, true, false, true>(a, stream)
                          : fa::launch_fa<T6, NQ, NK, false, false, true>(a, stream);
        }
    }
    // one workgroup per (b, h) and CU: only with probs and when the (b, h)
    // pairs fill the device (at B*H = 128, S = 256 the streaming kernel
    // measured 38.8 against 53.7 us for the drop-in); the resident kernel
    // writes no lse
    if (vec && probs && a.Sq >= kResidentMinSq && a.Sq <= kResidentMaxSq && !a.lse && a.D == 64 &&
        (int64_t)a.B * a.H >= device_cus() && fa::resident_lds_bytes<F32Traits<64, true>, 8>(a) != 0)
        return fa::launch_resident<F32Traits<64, true>, 8, 4>(a, causal, stream);
    switch (fa_f32_padded_dim(a.D)) {
        case 32:
            if (dp32_unsplit(a, causal, probs, vec)) return fa::launch_fa<F32Traits<32>, 2, 1, true, false, true>(a, stream);
            return launch_dp<32, 2, 2>(a, causal, probs, vec, stream);
        case 64:
            return dp64_narrow(a, causal) ? launch_dp<64, 4, 1, false>(a, causal, probs, vec, stream)
                                          : launch_dp<64, 4, 2>(a, causal, probs, vec, stream);
        case 128: return launch_dp<128, 8, 1>(a, causal, probs, vec, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hipgpt
