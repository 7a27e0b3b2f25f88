// fa_bf16.hip -- bf16-input / fp32-accumulate attention forward on gfx950.
//
// Same kernel body as the fp32 path (fa_kernel.h) with bf16 operand traits on
// v_mfma_f32_32x32x16_bf16:
//   * S^T = K Q^T: Q (bf16, unscaled) is the B operand in registers; lane
//     (c, h) takes d = h*D/2 + 8j .. +7 for step j, one ds_read_b128 of K row
//     c per MFMA.  The softmax scale is applied inside the exponent,
//     exp2(s*scale*log2e - m) as one FMA, so Q is never re-rounded to bf16
//     after scaling.
//   * O^T = V^T P^T: P is rounded to bf16 (RNE) straight from the score
//     accumulator; step s uses registers 8s .. 8s+7, i.e. keys
//     acc_key(8s + j, h).  V is staged row-major (one 16-byte LDS store per
//     chunk) and the same eight keys of a d column come back transposed by
//     two ds_read_b64_tr_b16.
//   * O is accumulated and written in fp32; probs (optional) are fp32.
// No reference kernel exists for this variant; it computes the reference's
// function on bf16-rounded inputs.
//
// MFMA 32x32x16 bf16 operand layout (lane l, c = l & 31, h = l >> 5):
//   A[m][k]: lane holds A[c][8h .. 8h+7]    B[k][n]: lane holds B[8h .. 8h+7][c]
//   D: as the f32 32x32 form (register r holds row 8*(r/4) + 4*h + r%4, col c)
#include "common.h"
#include "fa_kernel.h"
#include "kernels.h"

namespace hipgpt {

namespace {

using fa::BK;
typedef unsigned short u16;

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

template <int D_>
struct B16Traits {
    static constexpr int DP = D_;
    using elem = u16;
    using chunk = uint4;
    static constexpr int KSTR = DP + 8;  // rows 16*(DP/8+1) bytes apart
    // Row-major V rows: a pitch of DP + 16 (8 dwords past a multiple of 32)
    // puts the four 32-byte row pieces a 16-lane transpose read takes on
    // disjoint banks.
    static constexpr int VRP = DP + 16;
    static constexpr int KTILE = BK * KSTR;
    static constexpr int VTILE = BK * VRP;

    struct QReg {
        bf16x8 v[DP / 16];
    };

    template <bool VEC>
    __device__ __forceinline__ static void load_q(QReg& q, const u16* qrow, int hf, bool valid, int, float) {
        const u16* p = qrow + hf * (DP / 2);
#pragma unroll
        for (int s = 0; s < DP / 16; ++s)
            q.v[s] = as_bf16x8(valid ? *reinterpret_cast<const uint4*>(p + 8 * s) : uint4{0u, 0u, 0u, 0u});
    }

    __device__ __forceinline__ static float score_scale(float qscale) { return qscale; }
    __device__ __forceinline__ static chunk from_u32x4(u32x4 v) { return uint4{v[0], v[1], v[2], v[3]}; }

    template <bool VEC>
    __device__ __forceinline__ static chunk load_chunk(const u16* base, int64_t rowoff, int cc, int, bool ok) {
        return ok ? *reinterpret_cast<const uint4*>(base + rowoff + cc * 8) : uint4{0u, 0u, 0u, 0u};
    }
    __device__ __forceinline__ static void store_k_chunk(u16* Kt, int r, int cc, const chunk& v) {
        *reinterpret_cast<uint4*>(Kt + r * KSTR + cc * 8) = v;
    }
    // V stays row-major (key r, head dims 8cc .. 8cc+7); load_v transposes.
    __device__ __forceinline__ static void store_vt_chunk(u16* Vt, int r, int cc, const chunk& v) {
        *reinterpret_cast<uint4*>(Vt + r * VRP + cc * 8) = v;
    }

    __device__ __forceinline__ static floatx16 qk(const u16* Kt, const QReg& q, int c, int hf) {
        const u16* kr = Kt + c * KSTR + hf * (DP / 2);
        uint4 kv[DP / 16];
#pragma unroll
        for (int j = 0; j < DP / 16; ++j) kv[j] = *reinterpret_cast<const uint4*>(kr + 8 * j);
        floatx16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
        for (int j = 0; j < DP / 16; ++j) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kv[j]), q.v[j], s, 0, 0, 0);
        return s;
    }

    // V^T operands: step s of block db uses keys acc_key(8s + j, hf), i.e.
    // V[16s + 4hf + 0..3][db*32 + c] and V[16s + 8 + 4hf + 0..3][db*32 + c].
    struct VReg {
        uint4 v[DP / 32][2];
    };
    // ds_read_b64_tr_b16 (gfx950): in each 16-lane group, lane r supplies
    // the address of V[k0 + r/4][d0 + 4(r%4) .. +3] and lane i receives
    // V[k0 + 0..3][d0 + i] (lane layout checked on the MI355X).  Group
    // (hf, c/16) takes d0 = db*32 + (c & 16) and k0 = 16s + 4hf, +8 for the
    // second half of step s.
    __device__ __forceinline__ static void load_v(VReg& vr, const u16* Vt, int c, int hf) {
        const int r = c & 15;
#pragma unroll
        for (int db = 0; db < DP / 32; ++db) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const u16* p = Vt + (16 * s + 4 * hf + (r >> 2)) * VRP + db * 32 + (c & 16) + 4 * (r & 3);
                const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p));
                const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + 8 * VRP));
                const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
                vr.v[db][s] = uint4{l2.x, l2.y, h2.x, h2.y};
            }
        }
    }
    __device__ __forceinline__ static void pv(const VReg& vr, const floatx16& p, floatx16* o, int, int) {
        bf16x8 pb[2];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int j = 0; j < 8; ++j) pb[s][j] = (__bf16)p[8 * s + j];
#pragma unroll
        for (int db = 0; db < DP / 32; ++db)
#pragma unroll
            for (int s = 0; s < 2; ++s)
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(vr.v[db][s]), pb[s], o[db], 0, 0, 0);
    }
};

// Workgroup shape: 4 query sub-blocks (128 queries) share each K/V stage
// (bf16 tiles are short on the matrix cores, so the stage's loads, LDS
// stores and barrier are amortised over more work), each sub-block's keys
// split over 2 waves (4 x 2) or not (4 x 1).  A 4 x 1 workgroup takes half
// the CU, so the device holds twice as many, and where the 4 x 2 grid would
// need more than one round of resident workgroups the smaller workgroups
// fill the device better: without a causal mask when the grid exceeds the
// 4 x 2 slots, with one when it exceeds even the 4 x 1 slots (a causal grid
// that fits them at once measured slower: its longest rows, unsplit, set the
// end).  Cache-rotated, us, 4 x 2 -> 4 x 1 (G workgroups): non-causal
// B8 H12 S1024 D64 (G 768 against 512 4 x 2 slots) 47.5 -> 40.1, B4 H16
// S2048 D128 (G 1024 / 256) 209.8 -> 171.0; causal B4 H16 S2048 D128
// (G 1024 against 512 4 x 1 slots) 127.0 -> 110.1, B16 H12 S1024 D64
// (G 1536 / 1024) 58.9 -> 50.5.  Kept at 4 x 2: causal c3 (G 768 / 1024)
// 29.6 against 40.3, B4 H16 S2048 D64 (G 1024 / 1024) 56.9 / 72.1, B1 and
// B2 H12 S1024 D64 23.5 / 33.9 and 24.2 / 35.6, B32 H8 S256 D32 / D64
// 12.3 / 13.1 and 12.8 / 14.5; non-causal B32 H8 S256 D64 (G 512 / 512)
// 13.7 / 13.8.  2 x 1 and 8 x 1 measured between the two or slower.
constexpr int kNqs = 4;

template <int D>
hipError_t launch_d(const AttnArgs& a, bool causal, bool probs, hipStream_t s) {
    using T = B16Traits<D>;
    const int64_t grid = (int64_t)((a.Sq + kNqs * 32 - 1) / (kNqs * 32)) * a.B * a.H;
    const int slots = causal ? fa::fa_resident_slots<T, kNqs, 1, true, true>()
                             : fa::fa_resident_slots<T, kNqs, 2, false, true>();
    if (slots > 0 && grid > slots) return fa::launch_fa_flags<T, kNqs, 1, true>(a, causal, probs, s);
    return fa::launch_fa_flags<T, kNqs, 2, true>(a, causal, probs, s);
}

}  // namespace

bool fa_bf16_supported(int D) { return D == 32 || D == 64 || D == 128; }

hipError_t launch_fa_bf16(const AttnArgs& a, bool causal, hipStream_t stream) {
    const bool probs = a.probs != nullptr;
    switch (a.D) {
        case 32: return launch_d<32>(a, causal, probs, stream);
        case 64: return launch_d<64>(a, causal, probs, stream);
        case 128: return launch_d<128>(a, causal, probs, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hipgpt
