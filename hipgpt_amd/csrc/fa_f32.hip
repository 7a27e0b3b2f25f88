// fa_f32.hip -- exact fp32 attention forward on gfx950 MFMA.
//
// Replaces flash_attention_kernel<32|64> and multihead_attention_kernel_fallback
// (HipGPT src/hip_kernels.cpp:263-325, :329-402) for head dims up to 128.
//
// Work decomposition
//   * One workgroup = NW waves = NW*32 queries of one (batch, head).
//   * Key/value tiles of 32 rows are staged global -> registers -> LDS,
//     double buffered (one barrier per tile).  The next tile's global loads
//     are in flight while the current tile is on the matrix cores.  K is
//     kept row-major (one ds_read_b128 feeds four MFMAs); V is written
//     transposed so the P V operands are also ds_read_b128.
//   * Each wave computes S^T = K Q^T for its 32 queries with
//     v_mfma_f32_32x32x2_f32 (Q held in registers, pre-scaled by
//     scale*log2(e)); see fa_common.h for the accumulator layout.
//   * The exponentiated tile is directly the B operand of O^T = V^T P^T:
//     P never leaves registers.
//   * Causal: tiles above a wave's diagonal are skipped (wave-uniform), only
//     tiles crossing the diagonal are masked; query blocks are launched
//     longest-first and alternate blocks map their waves in reverse order so
//     a long and a short block sharing a CU load its SIMDs evenly.
//   * Without probs: single sweep with online softmax (O rescaled only when
//     some row max moved).  With probs (the legacy contract, normalised P
//     stored for the backward): sweep 1 finds the row max and sum, sweep 2
//     recomputes S, stores P = exp(s-m)/l once and accumulates P V -- the
//     reference's pass order without its S-sized per-thread scratch.
//
// MFMA 32x32x2 f32 operand layout (lane l, c = l & 31, h = l >> 5):
//   A[m][k]: lane holds A[c][h]          B[k][n]: lane holds B[h][c]
//   D[m][n]: register r holds D[8*(r/4) + 4*h + (r%4)][c]
#include "common.h"
#include "fa_common.h"
#include "kernels.h"

namespace hipgpt {

namespace {

using fa::BK;
using fa::QW;

template <int DP>
struct F32Tile {
    static constexpr int KSTR = DP + 4;   // K row pitch (floats): conflict-free ds_read_b128 rows
    static constexpr int VTP = BK + 4;    // V^T row pitch (floats)
    static constexpr int KSZ = BK * KSTR;
    static constexpr int VSZ = DP * VTP;
};

// Global -> register staging of one 32-row tile of K or V (fp32).
template <int DP, int NW, bool VEC>
struct TileLoader {
    static constexpr int NT = NW * 64;
    static constexpr int F4 = BK * DP / 4 / NT;  // float4 slots per thread
    static_assert(F4 >= 1 && (BK * DP / 4) % NT == 0, "tile must split evenly");
    floatx4 r[F4];

    __device__ __forceinline__ void load(const float* base, int64_t ts, int key0, int Sk, int D, int tid) {
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const int f = tid + i * NT;
            const int row = f / (DP / 4);
            const int c4 = f % (DP / 4);
            const int key = key0 + row;
            if (VEC) {
                if (key < Sk)
                    r[i] = *reinterpret_cast<const floatx4*>(base + (int64_t)key * ts + c4 * 4);
                else
                    r[i] = floatx4{0.f, 0.f, 0.f, 0.f};
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int d = c4 * 4 + j;
                    r[i][j] = (key < Sk && d < D) ? base[(int64_t)key * ts + d] : 0.f;
                }
            }
        }
    }
    // Row-major store: lds[row][d] with pitch KSTR.
    __device__ __forceinline__ void store_rows(float* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const int f = tid + i * NT;
            const int row = f / (DP / 4);
            const int c4 = f % (DP / 4);
            *reinterpret_cast<floatx4*>(lds + row * F32Tile<DP>::KSTR + c4 * 4) = r[i];
        }
    }
    // Transposed store: lds[d][row] with pitch VTP.
    __device__ __forceinline__ void store_cols(float* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const int f = tid + i * NT;
            const int row = f / (DP / 4);
            const int c4 = f % (DP / 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) lds[(c4 * 4 + j) * F32Tile<DP>::VTP + row] = r[i][j];
        }
    }
};

template <int DP, int NW, bool CAUSAL, bool PROBS, bool VEC>
__global__ __launch_bounds__(NW * 64) void fa_fwd_f32_kernel(AttnArgs a) {
    using T = F32Tile<DP>;
    constexpr int NDB = DP / 32;  // 32-row blocks of O^T

    __shared__ __attribute__((aligned(16))) float smem[2 * (T::KSZ + T::VSZ)];
    float* const Ks0 = smem;
    float* const Vs0 = smem + 2 * T::KSZ;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int c = lane & 31;
    const int hf = lane >> 5;

    const int BH = a.B * a.H;
    const int bh = blockIdx.x % BH;
    const int rank = blockIdx.x / BH;           // launch order of this query block
    const int qb = CAUSAL ? a.n_qblk - 1 - rank : rank;  // longest rows first
    const int wsub = (CAUSAL && (rank & 1)) ? NW - 1 - wave : wave;
    const int b = bh / a.H;
    const int h = bh % a.H;

    const int q0 = qb * (NW * QW);
    const int qw0 = q0 + wsub * QW;
    const int qi = qw0 + c;
    const int Sq = a.Sq, Sk = a.Sk, off = a.causal_off;

    const float* Qp = static_cast<const float*>(a.q) + b * a.q_bs + h * a.q_hs;
    const float* Kp = static_cast<const float*>(a.k) + b * a.k_bs + h * a.k_hs;
    const float* Vp = static_cast<const float*>(a.v) + b * a.v_bs + h * a.v_hs;

    const fa::TileRange tr = fa::tile_range<CAUSAL>(q0, qw0, NW * QW, Sq, Sk, off);
    const int ntiles = tr.ntiles, wtiles = tr.wtiles;

    // Q^T operand: lane (c, hf) holds Q[qi][hf*DP/2 + s], s = 0..DP/2-1.
    float qf[DP / 2];
    {
        const float* qrow = Qp + (int64_t)qi * a.q_ts + hf * (DP / 2);
        if (qi < Sq) {
            if (VEC) {
#pragma unroll
                for (int s = 0; s < DP / 2; s += 4) {
                    const floatx4 t = *reinterpret_cast<const floatx4*>(qrow + s);
#pragma unroll
                    for (int j = 0; j < 4; ++j) qf[s + j] = t[j] * a.qscale;
                }
            } else {
#pragma unroll
                for (int s = 0; s < DP / 2; ++s) qf[s] = (hf * (DP / 2) + s < a.D) ? qrow[s] * a.qscale : 0.f;
            }
        } else {
#pragma unroll
            for (int s = 0; s < DP / 2; ++s) qf[s] = 0.f;
        }
    }

    // S^T tile (32 keys x 32 queries) from the LDS K tile, masked.
    auto score_tile = [&](const float* Kt, int t) -> floatx16 {
        floatx16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.f;
        const float* kr = Kt + c * T::KSTR + hf * (DP / 2);
#pragma unroll
        for (int j = 0; j < DP / 2; j += 4) {
            const floatx4 kv = *reinterpret_cast<const floatx4*>(kr + j);
#pragma unroll
            for (int u = 0; u < 4; ++u) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[u], qf[j + u], s, 0, 0, 0);
        }
        if (tr.edge(t, Sk, CAUSAL, qw0, off)) fa::mask_tile<CAUSAL>(s, t * BK, hf, qi, Sk, off);
        return s;
    };

    floatx16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.f;

    // O^T += V^T P^T over one tile.  Lane (c, hf) of block db needs
    // V[acc_key(t, hf)][db*32 + c] for t = 0..15: four ds_read_b128 from V^T.
    auto pv_tile = [&](const float* Vt, const floatx16& p) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const float* vr = Vt + (db * 32 + c) * T::VTP + 4 * hf;
            floatx4 va[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) va[g] = *reinterpret_cast<const floatx4*>(vr + 8 * g);
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[g][u], p[4 * g + u], o[db], 0, 0, 0);
        }
    };

    float m_run = kMaxInit;  // running max (log2 domain)
    float l_run = 0.f;       // running sum

    TileLoader<DP, NW, VEC> kl, vl;

    if (!PROBS) {
        // ---------------- single sweep, online softmax ----------------
        if (ntiles > 0) {
            kl.load(Kp, a.k_ts, 0, Sk, a.D, tid);
            vl.load(Vp, a.v_ts, 0, Sk, a.D, tid);
            kl.store_rows(Ks0, tid);
            vl.store_cols(Vs0, tid);
        }
        __syncthreads();
        for (int t = 0; t < ntiles; ++t) {
            const int buf = t & 1;
            const bool more = t + 1 < ntiles;
            if (more) {
                kl.load(Kp, a.k_ts, (t + 1) * BK, Sk, a.D, tid);
                vl.load(Vp, a.v_ts, (t + 1) * BK, Sk, a.D, tid);
            }
            if (t < wtiles) {
                floatx16 s = score_tile(Ks0 + buf * T::KSZ, t);
                const float m_new = fmaxf(m_run, fa::tile_max(s));
                float ls = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    s[r] = fast_exp2(s[r] - m_new);
                    ls += s[r];
                }
                ls = fa::halves_sum(ls);
                if (__any(m_new != m_run)) {  // wave-uniform: rescale only when a max moved
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
        // ---------------- sweep 1: row max and row sum ----------------
        if (ntiles > 0) {
            kl.load(Kp, a.k_ts, 0, Sk, a.D, tid);
            kl.store_rows(Ks0, tid);
        }
        __syncthreads();
        for (int t = 0; t < ntiles; ++t) {
            const int buf = t & 1;
            const bool more = t + 1 < ntiles;
            if (more) kl.load(Kp, a.k_ts, (t + 1) * BK, Sk, a.D, tid);
            if (t < wtiles) {
                const floatx16 s = score_tile(Ks0 + buf * T::KSZ, t);
                const float m_new = fmaxf(m_run, fa::tile_max(s));
                float ls = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) ls += fast_exp2(s[r] - m_new);
                l_run = l_run * fast_exp2(m_run - m_new) + fa::halves_sum(ls);
                m_run = m_new;
            }
            if (more) kl.store_rows(Ks0 + (buf ^ 1) * T::KSZ, tid);
            __syncthreads();
        }
        // ------------- sweep 2: store P, accumulate P V -------------
        const float linv = 1.0f / fmaxf(l_run, 1e-20f);
        float* probs_bh = a.probs + (int64_t)bh * Sq * Sk;
        float* prow = probs_bh + (int64_t)qi * Sk;
        const bool pvec = (Sk & 3) == 0 && (reinterpret_cast<uintptr_t>(a.probs) & 15) == 0;
        if (ntiles > 0) {
            kl.load(Kp, a.k_ts, 0, Sk, a.D, tid);
            vl.load(Vp, a.v_ts, 0, Sk, a.D, tid);
            kl.store_rows(Ks0, tid);
            vl.store_cols(Vs0, tid);
        }
        __syncthreads();
        for (int t = 0; t < ntiles; ++t) {
            const int buf = t & 1;
            const bool more = t + 1 < ntiles;
            if (more) {
                kl.load(Kp, a.k_ts, (t + 1) * BK, Sk, a.D, tid);
                vl.load(Vp, a.v_ts, (t + 1) * BK, Sk, a.D, tid);
            }
            if (t < wtiles) {
                floatx16 s = score_tile(Ks0 + buf * T::KSZ, t);
#pragma unroll
                for (int r = 0; r < 16; ++r) s[r] = fast_exp2(s[r] - m_run) * linv;
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

    // ---------------- epilogue: O = O^T / l ----------------
    if (qi < Sq) {
        const float linv = PROBS ? 1.0f : 1.0f / fmaxf(l_run, 1e-20f);
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

template <int DP, int NW, bool CAUSAL, bool PROBS, bool VEC>
hipError_t launch_one(const AttnArgs& a, hipStream_t stream) {
    AttnArgs args = a;
    args.n_qblk = (a.Sq + NW * QW - 1) / (NW * QW);
    const int64_t grid = (int64_t)args.n_qblk * a.B * a.H;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((fa_fwd_f32_kernel<DP, NW, CAUSAL, PROBS, VEC>), dim3((unsigned)grid), dim3(NW * 64), 0,
                       stream, args);
    return hipGetLastError();
}

template <int DP, int NW>
hipError_t launch_dp(const AttnArgs& a, bool causal, bool probs, bool vec, hipStream_t s) {
    if (causal) {
        if (probs)
            return vec ? launch_one<DP, NW, true, true, true>(a, s) : launch_one<DP, NW, true, true, false>(a, s);
        return vec ? launch_one<DP, NW, true, false, true>(a, s) : launch_one<DP, NW, true, false, false>(a, s);
    }
    if (probs)
        return vec ? launch_one<DP, NW, false, true, true>(a, s) : launch_one<DP, NW, false, true, false>(a, s);
    return vec ? launch_one<DP, NW, false, false, true>(a, s) : launch_one<DP, NW, false, false, false>(a, s);
}

}  // namespace

int fa_f32_padded_dim(int D) {
    if (D <= 32) return 32;
    if (D <= 64) return 64;
    if (D <= 128) return 128;
    return 0;
}

hipError_t launch_fa_f32(const AttnArgs& a, bool causal, bool vec, hipStream_t stream) {
    const bool probs = a.probs != nullptr;
    switch (fa_f32_padded_dim(a.D)) {
        case 32: return launch_dp<32, 4>(a, causal, probs, vec, stream);
        case 64: return launch_dp<64, 4>(a, causal, probs, vec, stream);
        case 128: return launch_dp<128, 4>(a, causal, probs, vec, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hipgpt
