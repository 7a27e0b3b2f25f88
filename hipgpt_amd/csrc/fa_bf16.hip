// fa_bf16.hip -- bf16-input / fp32-accumulate attention forward on gfx950.
//
// Same decomposition as fa_f32.hip (see there and fa_common.h) with
// v_mfma_f32_32x32x16_bf16:
//   * S^T = K Q^T: Q (bf16, unscaled) is the B operand held in registers;
//     K tiles are row-major in LDS, one ds_read_b128 per MFMA.  The softmax
//     scale is applied inside the exponent, exp2(s*scale*log2e - m), so Q is
//     not re-rounded to bf16 after scaling.
//   * O^T = V^T P^T: P is rounded to bf16 (RNE) straight from the score
//     accumulator; V is stored transposed in LDS so each lane's eight keys
//     are two ds_read_b64.
//   * O is accumulated and written in fp32; probs (optional) are fp32.
// No reference kernel exists for this variant; it computes the reference's
// function on bf16-rounded inputs.
//
// MFMA 32x32x16 bf16 operand layout (lane l, c = l & 31, h = l >> 5):
//   A[m][k]: lane holds A[c][8h .. 8h+7]    B[k][n]: lane holds B[8h .. 8h+7][c]
//   D: as the f32 32x32 form (register r holds row 8*(r/4) + 4*h + r%4, col c)
// Step s of the P V product uses accumulator registers 8s .. 8s+7, i.e. keys
// acc_key(8s + j, h); V^T supplies the same eight keys in the same order.
#include "common.h"
#include "fa_common.h"
#include "kernels.h"

namespace hipgpt {

namespace {

using fa::BK;
using fa::QW;
typedef unsigned short u16;

template <int D>
struct B16Tile {
    static constexpr int KSTR = D + 8;  // K row pitch (bf16): rows 16*(D/8+1) bytes apart
    static constexpr int VTP = BK + 4;  // V^T row pitch (bf16): 72 bytes
    static constexpr int KSZ = BK * KSTR;
    static constexpr int VSZ = D * VTP;
};

// Global -> register staging of one 32-row bf16 tile (16-byte chunks).
template <int D, int NW>
struct B16Loader {
    static constexpr int NT = NW * 64;
    static constexpr int CH = BK * D / 8;  // 16-byte chunks per tile
    static constexpr int PER = (CH + NT - 1) / NT;
    uint4 r[PER];

    __device__ __forceinline__ void load(const u16* base, int64_t ts, int key0, int Sk, int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + i * NT;
            const int row = f / (D / 8);
            const int c8 = f % (D / 8);
            const int key = key0 + row;
            if (f < CH && key < Sk)
                r[i] = *reinterpret_cast<const uint4*>(base + (int64_t)key * ts + c8 * 8);
            else
                r[i] = uint4{0u, 0u, 0u, 0u};
        }
    }
    __device__ __forceinline__ void store_rows(u16* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + i * NT;
            if (f >= CH) break;
            const int row = f / (D / 8);
            const int c8 = f % (D / 8);
            *reinterpret_cast<uint4*>(lds + row * B16Tile<D>::KSTR + c8 * 8) = r[i];
        }
    }
    __device__ __forceinline__ void store_cols(u16* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + i * NT;
            if (f >= CH) break;
            const int row = f / (D / 8);
            const int c8 = f % (D / 8);
            const unsigned w[4] = {r[i].x, r[i].y, r[i].z, r[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lds[(c8 * 8 + 2 * j) * B16Tile<D>::VTP + row] = (u16)(w[j] & 0xffffu);
                lds[(c8 * 8 + 2 * j + 1) * B16Tile<D>::VTP + row] = (u16)(w[j] >> 16);
            }
        }
    }
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

template <int D, int NW, bool CAUSAL, bool PROBS>
__global__ __launch_bounds__(NW * 64) void fa_fwd_bf16_kernel(AttnArgs a) {
    using T = B16Tile<D>;
    constexpr int NDB = D / 32;
    constexpr int QS = D / 16;  // bf16x8 Q chunks per lane

    __shared__ __attribute__((aligned(16))) u16 smem[2 * (T::KSZ + T::VSZ)];
    u16* const Ks0 = smem;
    u16* const Vs0 = smem + 2 * T::KSZ;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int c = lane & 31;
    const int hf = lane >> 5;

    const int BH = a.B * a.H;
    const int bh = blockIdx.x % BH;
    const int rank = blockIdx.x / BH;
    const int qb = CAUSAL ? a.n_qblk - 1 - rank : rank;
    const int wsub = (CAUSAL && (rank & 1)) ? NW - 1 - wave : wave;
    const int b = bh / a.H;
    const int h = bh % a.H;

    const int q0 = qb * (NW * QW);
    const int qw0 = q0 + wsub * QW;
    const int qi = qw0 + c;
    const int Sq = a.Sq, Sk = a.Sk, off = a.causal_off;
    const float sc = a.qscale;

    const u16* Qp = static_cast<const u16*>(a.q) + b * a.q_bs + h * a.q_hs;
    const u16* Kp = static_cast<const u16*>(a.k) + b * a.k_bs + h * a.k_hs;
    const u16* Vp = static_cast<const u16*>(a.v) + b * a.v_bs + h * a.v_hs;

    const fa::TileRange tr = fa::tile_range<CAUSAL>(q0, qw0, NW * QW, Sq, Sk, off);
    const int ntiles = tr.ntiles, wtiles = tr.wtiles;

    // Q^T operand: lane (c, hf) chunk s holds Q[qi][hf*D/2 + 8s .. +7].
    bf16x8 qf[QS];
    {
        const u16* qrow = Qp + (int64_t)qi * a.q_ts + hf * (D / 2);
#pragma unroll
        for (int s = 0; s < QS; ++s)
            qf[s] = as_bf16x8(qi < Sq ? *reinterpret_cast<const uint4*>(qrow + 8 * s) : uint4{0u, 0u, 0u, 0u});
    }

    // Raw (unscaled) S^T tile, masked with -inf.
    auto score_tile = [&](const u16* Kt, int t) -> floatx16 {
        floatx16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.f;
        const u16* kr = Kt + c * T::KSTR + hf * (D / 2);
#pragma unroll
        for (int j = 0; j < QS; ++j) {
            const bf16x8 kv = as_bf16x8(*reinterpret_cast<const uint4*>(kr + 8 * j));
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kv, qf[j], s, 0, 0, 0);
        }
        if (tr.edge(t, Sk, CAUSAL, qw0, off)) fa::mask_tile<CAUSAL>(s, t * BK, hf, qi, Sk, off);
        return s;
    };

    floatx16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.f;

    auto pv_tile = [&](const u16* Vt, const floatx16& p) {
        bf16x8 pb[2];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int j = 0; j < 8; ++j) pb[s][j] = (__bf16)p[8 * s + j];
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const u16* vr = Vt + (db * 32 + c) * T::VTP + 4 * hf;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const uint2 lo = *reinterpret_cast<const uint2*>(vr + 16 * s);
                const uint2 hi = *reinterpret_cast<const uint2*>(vr + 16 * s + 8);
                const bf16x8 va = as_bf16x8(uint4{lo.x, lo.y, hi.x, hi.y});
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[s], o[db], 0, 0, 0);
            }
        }
    };

    float m_run = kMaxInit;  // running max of s*sc (log2 domain)
    float l_run = 0.f;

    B16Loader<D, NW> kl, vl;

    if (!PROBS) {
        if (ntiles > 0) {
            kl.load(Kp, a.k_ts, 0, Sk, tid);
            vl.load(Vp, a.v_ts, 0, Sk, tid);
            kl.store_rows(Ks0, tid);
            vl.store_cols(Vs0, tid);
        }
        __syncthreads();
        for (int t = 0; t < ntiles; ++t) {
            const int buf = t & 1;
            const bool more = t + 1 < ntiles;
            if (more) {
                kl.load(Kp, a.k_ts, (t + 1) * BK, Sk, tid);
                vl.load(Vp, a.v_ts, (t + 1) * BK, Sk, tid);
            }
            if (t < wtiles) {
                floatx16 s = score_tile(Ks0 + buf * T::KSZ, t);
                const float m_new = fmaxf(m_run, fa::tile_max(s) * sc);
                float ls = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    s[r] = fast_exp2(fmaf(s[r], sc, -m_new));
                    ls += s[r];
                }
                ls = fa::halves_sum(ls);
                if (__any(m_new != m_run)) {
                    const float alpha = fast_exp2(m_run - m_new);
                    l_run *= alpha;
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
#pragma unroll
                        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
                }
                l_run += ls;
                m_run = m_new;
                pv_tile(Vs0 + buf * T::VSZ, s);
            }
            if (more) {
                kl.store_rows(Ks0 + (buf ^ 1) * T::KSZ, tid);
                vl.store_cols(Vs0 + (buf ^ 1) * T::VSZ, tid);
            }
            __syncthreads();
        }
    } else {
        if (ntiles > 0) {
            kl.load(Kp, a.k_ts, 0, Sk, tid);
            kl.store_rows(Ks0, tid);
        }
        __syncthreads();
        for (int t = 0; t < ntiles; ++t) {
            const int buf = t & 1;
            const bool more = t + 1 < ntiles;
            if (more) kl.load(Kp, a.k_ts, (t + 1) * BK, Sk, tid);
            if (t < wtiles) {
                const floatx16 s = score_tile(Ks0 + buf * T::KSZ, t);
                const float m_new = fmaxf(m_run, fa::tile_max(s) * sc);
                float ls = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) ls += fast_exp2(fmaf(s[r], sc, -m_new));
                l_run = l_run * fast_exp2(m_run - m_new) + fa::halves_sum(ls);
                m_run = m_new;
            }
            if (more) kl.store_rows(Ks0 + (buf ^ 1) * T::KSZ, tid);
            __syncthreads();
        }
        const float linv = 1.0f / fmaxf(l_run, 1e-20f);
        float* probs_bh = a.probs + (int64_t)bh * Sq * Sk;
        float* prow = probs_bh + (int64_t)qi * Sk;
        const bool pvec = (Sk & 3) == 0 && (reinterpret_cast<uintptr_t>(a.probs) & 15) == 0;
        if (ntiles > 0) {
            kl.load(Kp, a.k_ts, 0, Sk, tid);
            vl.load(Vp, a.v_ts, 0, Sk, tid);
            kl.store_rows(Ks0, tid);
            vl.store_cols(Vs0, tid);
        }
        __syncthreads();
        for (int t = 0; t < ntiles; ++t) {
            const int buf = t & 1;
            const bool more = t + 1 < ntiles;
            if (more) {
                kl.load(Kp, a.k_ts, (t + 1) * BK, Sk, tid);
                vl.load(Vp, a.v_ts, (t + 1) * BK, Sk, tid);
            }
            if (t < wtiles) {
                floatx16 s = score_tile(Ks0 + buf * T::KSZ, t);
#pragma unroll
                for (int r = 0; r < 16; ++r) s[r] = fast_exp2(fmaf(s[r], sc, -m_run)) * linv;
                if (qi < Sq) fa::store_probs_tile(prow, s, t * BK, hf, Sk, pvec);
                pv_tile(Vs0 + buf * T::VSZ, s);
            }
            if (more) {
                kl.store_rows(Ks0 + (buf ^ 1) * T::KSZ, tid);
                vl.store_cols(Vs0 + (buf ^ 1) * T::VSZ, tid);
            }
            __syncthreads();
        }
        if (CAUSAL && qw0 < Sq) fa::zero_probs_tail(probs_bh, qw0, Sq, Sk, wtiles * BK, lane, pvec);
    }

    if (qi < Sq) {
        const float linv = PROBS ? 1.0f : 1.0f / fmaxf(l_run, 1e-20f);
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

template <int D, int NW, bool CAUSAL, bool PROBS>
hipError_t launch_one(const AttnArgs& a, hipStream_t stream) {
    AttnArgs args = a;
    args.n_qblk = (a.Sq + NW * QW - 1) / (NW * QW);
    const int64_t grid = (int64_t)args.n_qblk * a.B * a.H;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((fa_fwd_bf16_kernel<D, NW, CAUSAL, PROBS>), dim3((unsigned)grid), dim3(NW * 64), 0, stream,
                       args);
    return hipGetLastError();
}

template <int D, int NW>
hipError_t launch_d(const AttnArgs& a, bool causal, bool probs, hipStream_t s) {
    if (causal) return probs ? launch_one<D, NW, true, true>(a, s) : launch_one<D, NW, true, false>(a, s);
    return probs ? launch_one<D, NW, false, true>(a, s) : launch_one<D, NW, false, false>(a, s);
}

}  // namespace

bool fa_bf16_supported(int D) { return D == 32 || D == 64 || D == 128; }

hipError_t launch_fa_bf16(const AttnArgs& a, bool causal, hipStream_t stream) {
    const bool probs = a.probs != nullptr;
    switch (a.D) {
        case 32: return launch_d<32, 4>(a, causal, probs, stream);
        case 64: return launch_d<64, 4>(a, causal, probs, stream);
        case 128: return launch_d<128, 4>(a, causal, probs, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hipgpt
