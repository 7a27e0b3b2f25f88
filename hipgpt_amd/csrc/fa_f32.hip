// fa_f32.hip -- exact fp32 attention forward on gfx950 MFMA.
//
// Replaces flash_attention_kernel<32|64> and multihead_attention_kernel_fallback
// (HipGPT src/hip_kernels.cpp:263-325, :329-402) for head dims up to 128.
//
// Work decomposition
//   * One workgroup = NW waves = NW*32 queries of one (batch, head).
//   * Key/value tiles of 32 rows are staged global -> registers -> LDS,
//     double buffered (one barrier per tile).  The next tile's global loads
//     are in flight while the current tile is on the matrix cores.
//   * Each wave computes S^T = K Q^T for its 32 queries with
//     v_mfma_f32_32x32x2_f32 (Q held in registers, pre-scaled by
//     scale*log2(e)), so every lane owns one query column and 16 key rows of
//     the 32x32 score tile.  Row max / row sum need 15 in-lane ops plus one
//     exchange with the other wave half.
//   * The exponentiated tile is already laid out as the B operand of
//     O^T = V^T P^T, so P never leaves registers: the key order of the
//     accumulator's 16 registers is reproduced when V is read from LDS.
//   * Causal: tiles above a wave's diagonal are skipped (wave-uniform), only
//     tiles crossing the diagonal are masked; query blocks are launched
//     longest-first.
//   * Without probs: single sweep with online softmax.  With probs (the
//     legacy contract, normalised P stored for the backward): sweep 1 finds
//     the row max and sum, sweep 2 recomputes S, stores P = exp(s-m)/l once
//     and accumulates P V -- the reference's pass order without its S-sized
//     per-thread scratch.
//
// MFMA 32x32x2 f32 operand layout (lane l, c = l & 31, h = l >> 5):
//   A[m][k]: lane holds A[c][h]          B[k][n]: lane holds B[h][c]
//   D[m][n]: register r holds D[8*(r/4) + 4*h + (r%4)][c]
#include "common.h"
#include "kernels.h"

namespace hipgpt {

namespace {

constexpr int BK = 32;  // keys per tile

template <int DP>
struct F32Tile {
    static constexpr int KSTR = DP + 4;  // LDS row pitch of K (ds_read_b128 rows)
    static constexpr int VSTR = DP + 8;  // LDS row pitch of V (two half-wave rows)
    static constexpr int KSZ = BK * KSTR;
    static constexpr int VSZ = BK * VSTR;
};

// Key (within the tile) held by accumulator register r of lane half h.
__device__ __forceinline__ int acc_key(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

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
    __device__ __forceinline__ void store(float* lds, int pitch, int tid) const {
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const int f = tid + i * NT;
            const int row = f / (DP / 4);
            const int c4 = f % (DP / 4);
            *reinterpret_cast<floatx4*>(lds + row * pitch + c4 * 4) = r[i];
        }
    }
};

template <int DP, int NW, bool CAUSAL, bool PROBS, bool VEC>
__global__ __launch_bounds__(NW * 64) void fa_fwd_f32_kernel(AttnArgs a) {
    using T = F32Tile<DP>;
    constexpr int QW = 32;  // queries per wave
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
    int qb = blockIdx.x / BH;
    if (CAUSAL) qb = a.n_qblk - 1 - qb;  // longest rows first
    const int b = bh / a.H;
    const int h = bh % a.H;

    const int q0 = qb * (NW * QW);
    const int qw0 = q0 + wave * QW;
    const int qi = qw0 + c;
    const int Sq = a.Sq, Sk = a.Sk;

    const float* Qp = static_cast<const float*>(a.q) + b * a.q_bs + h * a.q_hs;
    const float* Kp = static_cast<const float*>(a.k) + b * a.k_bs + h * a.k_hs;
    const float* Vp = static_cast<const float*>(a.v) + b * a.v_bs + h * a.v_hs;

    // Keys the workgroup needs, and keys this wave needs.
    int kend = Sk;
    if (CAUSAL) kend = min(Sk, min(q0 + NW * QW, Sq) + a.causal_off);
    const int ntiles = (kend + BK - 1) / BK;
    int wkend = Sk;
    if (CAUSAL) wkend = min(Sk, min(qw0 + QW, Sq) + a.causal_off);
    const int wtiles = (qw0 < Sq) ? (wkend + BK - 1) / BK : 0;

    // Q^T operand: lane (c, hf) holds Q[qi][hf*DP/2 + s], s = 0..DP/2-1.
    float qf[DP / 2];
    {
        const float* qrow = Qp + (int64_t)qi * a.q_ts + hf * (DP / 2);
        if (qi < Sq) {
            if (VEC) {
#pragma unroll
                for (int s = 0; s < DP / 2; s += 4) {
                    floatx4 t = *reinterpret_cast<const floatx4*>(qrow + s);
                    qf[s] = t[0] * a.qscale;
                    qf[s + 1] = t[1] * a.qscale;
                    qf[s + 2] = t[2] * a.qscale;
                    qf[s + 3] = t[3] * a.qscale;
                }
            } else {
#pragma unroll
                for (int s = 0; s < DP / 2; ++s)
                    qf[s] = (hf * (DP / 2) + s < a.D) ? qrow[s] * a.qscale : 0.f;
            }
        } else {
#pragma unroll
            for (int s = 0; s < DP / 2; ++s) qf[s] = 0.f;
        }
    }

    // S^T tile (32 keys x 32 queries) from the LDS K tile.
    auto score_tile = [&](const float* Kt, int tb) -> floatx16 {
        floatx16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.f;
        const float* kr = Kt + c * T::KSTR + hf * (DP / 2);
#pragma unroll
        for (int j = 0; j < DP / 2; j += 4) {
            const floatx4 kv = *reinterpret_cast<const floatx4*>(kr + j);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[0], qf[j], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[1], qf[j + 1], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[2], qf[j + 2], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[3], qf[j + 3], s, 0, 0, 0);
        }
        // Mask keys past Sk and, causally, past the query's diagonal.
        const bool edge = (tb + BK > Sk) || (CAUSAL && tb + BK - 1 > qw0 + a.causal_off);
        if (edge) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = tb + acc_key(r, hf);
                const bool vis = key < Sk && (!CAUSAL || key <= qi + a.causal_off);
                if (!vis) s[r] = kNegInf;
            }
        }
        return s;
    };

    floatx16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.f;

    // O^T += V^T P^T over one tile; p is the exponentiated score tile.
    auto pv_tile = [&](const float* Vt, const floatx16& p) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const float* vc = Vt + db * 32 + c;
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const float va = vc[acc_key(t, hf) * T::VSTR];
                o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va, p[t], o[db], 0, 0, 0);
            }
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
            kl.store(Ks0, T::KSTR, tid);
            vl.store(Vs0, T::VSTR, tid);
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
                floatx16 s = score_tile(Ks0 + buf * T::KSZ, t * BK);
                float mt = s[0];
#pragma unroll
                for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
                mt = fmaxf(mt, xor32(mt));
                const float m_new = fmaxf(m_run, mt);
                const float alpha = fast_exp2(m_run - m_new);
                float ls = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    s[r] = fast_exp2(s[r] - m_new);
                    ls += s[r];
                }
                ls += xor32(ls);
                l_run = l_run * alpha + ls;
                m_run = m_new;
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
                pv_tile(Vs0 + buf * T::VSZ, s);
            }
            if (more) {
                kl.store(Ks0 + (buf ^ 1) * T::KSZ, T::KSTR, tid);
                vl.store(Vs0 + (buf ^ 1) * T::VSZ, T::VSTR, tid);
            }
            __syncthreads();
        }
    } else {
        // ---------------- sweep 1: row max and row sum ----------------
        if (ntiles > 0) {
            kl.load(Kp, a.k_ts, 0, Sk, a.D, tid);
            kl.store(Ks0, T::KSTR, tid);
        }
        __syncthreads();
        for (int t = 0; t < ntiles; ++t) {
            const int buf = t & 1;
            const bool more = t + 1 < ntiles;
            if (more) kl.load(Kp, a.k_ts, (t + 1) * BK, Sk, a.D, tid);
            if (t < wtiles) {
                floatx16 s = score_tile(Ks0 + buf * T::KSZ, t * BK);
                float mt = s[0];
#pragma unroll
                for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
                mt = fmaxf(mt, xor32(mt));
                const float m_new = fmaxf(m_run, mt);
                float ls = 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) ls += fast_exp2(s[r] - m_new);
                ls += xor32(ls);
                l_run = l_run * fast_exp2(m_run - m_new) + ls;
                m_run = m_new;
            }
            if (more) kl.store(Ks0 + (buf ^ 1) * T::KSZ, T::KSTR, tid);
            __syncthreads();
        }
        // ------------- sweep 2: store P, accumulate P V -------------
        const float linv = 1.0f / fmaxf(l_run, 1e-20f);
        float* prow = a.probs + ((int64_t)bh * Sq + qi) * (int64_t)Sk;
        const bool pvec = (Sk & 3) == 0;
        if (ntiles > 0) {
            kl.load(Kp, a.k_ts, 0, Sk, a.D, tid);
            vl.load(Vp, a.v_ts, 0, Sk, a.D, tid);
            kl.store(Ks0, T::KSTR, tid);
            vl.store(Vs0, T::VSTR, tid);
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
                const int tb = t * BK;
                floatx16 s = score_tile(Ks0 + buf * T::KSZ, tb);
#pragma unroll
                for (int r = 0; r < 16; ++r) s[r] = fast_exp2(s[r] - m_run) * linv;
                if (qi < Sq) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int k0 = tb + 8 * g + 4 * hf;
                        if (pvec && k0 + 3 < Sk) {
                            *reinterpret_cast<floatx4*>(prow + k0) =
                                floatx4{s[4 * g], s[4 * g + 1], s[4 * g + 2], s[4 * g + 3]};
                        } else {
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                                if (k0 + j < Sk) prow[k0 + j] = s[4 * g + j];
                        }
                    }
                }
                pv_tile(Vs0 + buf * T::VSZ, s);
            }
            if (more) {
                kl.store(Ks0 + (buf ^ 1) * T::KSZ, T::KSTR, tid);
                vl.store(Vs0 + (buf ^ 1) * T::VSZ, T::VSTR, tid);
            }
            __syncthreads();
        }
        // Causal: zero the probs of keys past this wave's last computed tile.
        if (CAUSAL && qw0 < Sq) {
            const int z0 = wtiles * BK;
            for (int r = 0; r < QW; ++r) {
                const int q = qw0 + r;
                if (q >= Sq) break;
                float* pr = a.probs + ((int64_t)bh * Sq + q) * (int64_t)Sk;
                if (pvec) {
                    for (int k = z0 + lane * 4; k < Sk; k += 256)
                        *reinterpret_cast<floatx4*>(pr + k) = floatx4{0.f, 0.f, 0.f, 0.f};
                } else {
                    for (int k = z0 + lane; k < Sk; k += 64) pr[k] = 0.f;
                }
            }
        }
        l_run = 1.0f;  // P was already normalised
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
                const floatx4 v = {o[db][4 * g] * linv, o[db][4 * g + 1] * linv,
                                   o[db][4 * g + 2] * linv, o[db][4 * g + 3] * linv};
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
    args.n_qblk = (a.Sq + NW * 32 - 1) / (NW * 32);
    const int64_t grid = (int64_t)args.n_qblk * a.B * a.H;
    if (grid <= 0 || grid > 0x7fffffff) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((fa_fwd_f32_kernel<DP, NW, CAUSAL, PROBS, VEC>), dim3((unsigned)grid),
                       dim3(NW * 64), 0, stream, args);
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
