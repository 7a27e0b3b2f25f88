// bwd.hip -- attention backward for HipGPT's probs contract, on gfx950 MFMA.
//
// Replaces multihead_attention_backward_kernel + launcher (HipGPT
// src/hip_kernels.cpp:1159-1272).  Same inputs and outputs: dO [B*S][E], the
// planar Q|K|V buffer, the forward's normalised probs P [B][H][S][S]; writes
// the planar dQ|dK|dV buffer.  Math per (b, h), scale c = 1/sqrt(D):
//   Dq_i = sum_j P_ij (dO_i . V_j)       (= dO_i . (P V)_i)
//   dS   = P o (dO V^T - Dq)
//   dQ = c dS K,   dK = c dS^T Q,   dV = P^T dO
// Head dims 32 and 64 with 16-byte aligned rows run the LDS-tiled kernels of
// bwd_tiled.h; the kernels below serve every other problem.  Two kernels,
// every gradient element written exactly once (no atomics, no memset):
//   * query-stationary (one wave per 32 queries): pass 1 forms (P V)_i on
//     MFMA and Dq_i = dO_i . (P V)_i (stored to a B*H*S workspace); pass 2
//     forms dP^T = V dO^T, dS, and dQ^T += K^T dS^T.
//   * key-stationary (one wave per 32 keys, V_j held in registers): per query
//     tile, dP = dO V^T lands with one key per lane and the tile's queries in
//     the accumulator's register order -- exactly the B operand layout of
//     dV^T += dO^T P and dK^T += Q^T dS, so P and dS never leave registers.
// P, dO, Q, K, V tiles are read straight from global memory (L2-resident per
// (b, h)) in the operand layouts; the fa_common.h accumulator layout applies.
// Causal (extended API only) skips tiles of P that lie wholly above the
// diagonal, where a causal forward wrote zeros.
#include "bwd_bh.h"
#include "bwd_bh64.h"
#include "bwd_tiled.h"
#include "bwd_wide.h"
#include "common.h"
#include "fa_common.h"
#include "kernels.h"

namespace hipgpt {

namespace {

using fa::acc_key;
using fa::halves_sum;

template <int DP>
__global__ __launch_bounds__(256) void bwd_dq_kernel(BwdArgs a) {
    constexpr int NDB = DP / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 31, hf = lane >> 5;
    const int nq = (a.S + 31) / 32;
    const int64_t blk = (int64_t)blockIdx.x * 4 + wave;
    if (blk >= (int64_t)a.B * a.H * nq) return;  // wave-uniform
    const int qt = (int)(blk % nq);
    const int bh = (int)(blk / nq);
    const int b = bh / a.H, h = bh % a.H;
    const int S = a.S, D = a.D;
    const int qi = qt * 32 + c;
    const int64_t base = (int64_t)b * a.bs + (int64_t)h * a.hs;
    const float* K = a.k + base;
    const float* V = a.v + base;
    const float* G = a.go + base;
    const float* P = a.probs + (int64_t)bh * S * S;
    const int nk = a.causal ? min((qt * 32 + 31) / 32 + 1, (S + 31) / 32) : (S + 31) / 32;

    // P^T operand of a key tile: register r <-> key kt*32 + acc_key(r, hf).
    auto load_p = [&](int kt, floatx16& p) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int j = kt * 32 + acc_key(r, hf);
            p[r] = (qi < S && j < S) ? P[(int64_t)qi * S + j] : 0.f;
        }
    };
    // A operand X^T[d][key] of block db: lane (c, hf) step t needs X[key(t)][db*32 + c].
    auto load_colT = [&](const float* X, int kt, int db, float* dst) {
        const int d = db * 32 + c;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int j = kt * 32 + acc_key(t, hf);
            dst[t] = (j < S && d < D) ? X[(int64_t)j * a.ts + d] : 0.f;
        }
    };

    // ---- pass 1: (P V)_i, then Dq_i = dO_i . (P V)_i ----
    floatx16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
    for (int kt = 0; kt < nk; ++kt) {
        floatx16 p;
        load_p(kt, p);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            float va[16];
            load_colT(V, kt, db, va);
#pragma unroll
            for (int t = 0; t < 16; ++t) o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[t], p[t], o[db], 0, 0, 0);
        }
    }
    float dq_dot = 0.f;
    if (qi < S) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int d = db * 32 + acc_key(r, hf);
                if (d < D) dq_dot = fmaf(G[(int64_t)qi * a.ts + d], o[db][r], dq_dot);
            }
    }
    dq_dot = halves_sum(dq_dot);
    if (hf == 0 && qi < S) a.dvec[(int64_t)bh * S + qi] = dq_dot;

    // ---- pass 2: dP^T = V dO^T, dS, dQ^T += K^T dS^T ----
    float gf[DP / 2];  // B operand: dO[qi][hf*DP/2 + s]
#pragma unroll
    for (int s = 0; s < DP / 2; ++s) {
        const int d = hf * (DP / 2) + s;
        gf[s] = (qi < S && d < D) ? G[(int64_t)qi * a.ts + d] : 0.f;
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.f;  // now dQ^T
    for (int kt = 0; kt < nk; ++kt) {
        const int key = kt * 32 + c;
        floatx16 dp;
#pragma unroll
        for (int r = 0; r < 16; ++r) dp[r] = 0.f;
#pragma unroll
        for (int s = 0; s < DP / 2; ++s) {
            const int d = hf * (DP / 2) + s;
            const float vv = (key < S && d < D) ? V[(int64_t)key * a.ts + d] : 0.f;
            dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, gf[s], dp, 0, 0, 0);
        }
        floatx16 p;
        load_p(kt, p);
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = p[r] * (dp[r] - dq_dot);  // dS^T
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            float ka[16];
            load_colT(K, kt, db, ka);
#pragma unroll
            for (int t = 0; t < 16; ++t) o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[t], p[t], o[db], 0, 0, 0);
        }
    }
    if (qi < S) {
        float* dq = a.dq + base + (int64_t)qi * a.ts;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int d = db * 32 + acc_key(r, hf);
                if (d < D) dq[d] = o[db][r] * a.scale;
            }
    }
}

template <int DP>
__global__ __launch_bounds__(256) void bwd_dkdv_kernel(BwdArgs a) {
    constexpr int NDB = DP / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 31, hf = lane >> 5;
    const int nk = (a.S + 31) / 32;
    const int64_t blk = (int64_t)blockIdx.x * 4 + wave;
    if (blk >= (int64_t)a.B * a.H * nk) return;  // wave-uniform
    const int kt = (int)(blk % nk);
    const int bh = (int)(blk / nk);
    const int b = bh / a.H, h = bh % a.H;
    const int S = a.S, D = a.D;
    const int kj = kt * 32 + c;
    const int64_t base = (int64_t)b * a.bs + (int64_t)h * a.hs;
    const float* Q = a.q + base;
    const float* V = a.v + base;
    const float* G = a.go + base;
    const float* P = a.probs + (int64_t)bh * S * S;
    const float* Dv = a.dvec + (int64_t)bh * S;
    const int nq = (S + 31) / 32;
    const int it0 = a.causal ? kt : 0;  // query tiles wholly above the diagonal hold P = 0

    float vf[DP / 2];  // B operand V^T: lane (c = key, hf) holds V[kj][hf*DP/2 + s]
#pragma unroll
    for (int s = 0; s < DP / 2; ++s) {
        const int d = hf * (DP / 2) + s;
        vf[s] = (kj < S && d < D) ? V[(int64_t)kj * a.ts + d] : 0.f;
    }
    floatx16 dk[NDB], dv[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dk[db][r] = dv[db][r] = 0.f;

    for (int it = it0; it < nq; ++it) {
        const int qrow = it * 32 + c;  // A operand row for dP
        floatx16 dp;
#pragma unroll
        for (int r = 0; r < 16; ++r) dp[r] = 0.f;
#pragma unroll
        for (int s = 0; s < DP / 2; ++s) {
            const int d = hf * (DP / 2) + s;
            const float g = (qrow < S && d < D) ? G[(int64_t)qrow * a.ts + d] : 0.f;
            dp = __builtin_amdgcn_mfma_f32_32x32x2f32(g, vf[s], dp, 0, 0, 0);
        }
        // P and Dq in the same layout: register r <-> query it*32 + acc_key(r, hf)
        floatx16 p, ds;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = it * 32 + acc_key(r, hf);
            const bool ok = i < S && kj < S;
            p[r] = ok ? P[(int64_t)i * S + kj] : 0.f;
            const float dqd = i < S ? Dv[i] : 0.f;
            ds[r] = p[r] * (dp[r] - dqd);
        }
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const int d = db * 32 + c;
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int i = it * 32 + acc_key(t, hf);
                const bool ok = i < S && d < D;
                const float ga = ok ? G[(int64_t)i * a.ts + d] : 0.f;
                const float qa = ok ? Q[(int64_t)i * a.ts + d] : 0.f;
                dv[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(ga, p[t], dv[db], 0, 0, 0);
                dk[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(qa, ds[t], dk[db], 0, 0, 0);
            }
        }
    }
    if (kj < S) {
        float* dkr = a.dk + base + (int64_t)kj * a.ts;
        float* dvr = a.dv + base + (int64_t)kj * a.ts;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int d = db * 32 + acc_key(r, hf);
                if (d < D) {
                    dkr[d] = dk[db][r] * a.scale;
                    dvr[d] = dv[db][r];
                }
            }
    }
}

// Any head dim: one thread per (token, head), the reference's two passes,
// with dK / dV gathered per key (no atomics): thread (b, j, h) sums over i.
__global__ __launch_bounds__(256) void bwd_generic_q_kernel(BwdArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = (int64_t)a.B * a.H * a.S;
    if (idx >= n) return;
    const int i = (int)(idx % a.S);
    const int bh = (int)(idx / a.S);
    const int b = bh / a.H, h = bh % a.H;
    const int64_t base = (int64_t)b * a.bs + (int64_t)h * a.hs;
    const float* g = a.go + base + (int64_t)i * a.ts;
    const float* prow = a.probs + ((int64_t)bh * a.S + i) * a.S;
    float ws = 0.f;
    for (int j = 0; j < a.S; ++j) {
        const float* v = a.v + base + (int64_t)j * a.ts;
        float vd = 0.f;
        for (int d = 0; d < a.D; ++d) vd = fmaf(g[d], v[d], vd);
        ws = fmaf(prow[j], vd, ws);
    }
    a.dvec[idx] = ws;
    float* dq = a.dq + base + (int64_t)i * a.ts;
    for (int d = 0; d < a.D; ++d) dq[d] = 0.f;
    for (int j = 0; j < a.S; ++j) {
        const float* v = a.v + base + (int64_t)j * a.ts;
        const float* k = a.k + base + (int64_t)j * a.ts;
        float vd = 0.f;
        for (int d = 0; d < a.D; ++d) vd = fmaf(g[d], v[d], vd);
        const float gs = prow[j] * (vd - ws) * a.scale;
        for (int d = 0; d < a.D; ++d) dq[d] = fmaf(gs, k[d], dq[d]);
    }
}

__global__ __launch_bounds__(256) void bwd_generic_kv_kernel(BwdArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = (int64_t)a.B * a.H * a.S;
    if (idx >= n) return;
    const int j = (int)(idx % a.S);
    const int bh = (int)(idx / a.S);
    const int b = bh / a.H, h = bh % a.H;
    const int64_t base = (int64_t)b * a.bs + (int64_t)h * a.hs;
    const float* v = a.v + base + (int64_t)j * a.ts;
    float* dk = a.dk + base + (int64_t)j * a.ts;
    float* dv = a.dv + base + (int64_t)j * a.ts;
    for (int d = 0; d < a.D; ++d) dk[d] = dv[d] = 0.f;
    for (int i = 0; i < a.S; ++i) {
        const float* g = a.go + base + (int64_t)i * a.ts;
        const float* q = a.q + base + (int64_t)i * a.ts;
        const float pij = a.probs[((int64_t)bh * a.S + i) * a.S + j];
        float vd = 0.f;
        for (int d = 0; d < a.D; ++d) vd = fmaf(g[d], v[d], vd);
        const float gs = pij * (vd - a.dvec[(int64_t)bh * a.S + i]) * a.scale;
        for (int d = 0; d < a.D; ++d) {
            dv[d] = fmaf(pij, g[d], dv[d]);
            dk[d] = fmaf(gs, q[d], dk[d]);
        }
    }
}

template <int DP>
hipError_t launch_dp(const BwdArgs& a, hipStream_t s) {
    const int64_t blocks = ((int64_t)a.B * a.H * ((a.S + 31) / 32) + 3) / 4;
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(bwd_dq_kernel<DP>, dim3((unsigned)blocks), dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(bwd_dkdv_kernel<DP>, dim3((unsigned)blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

// Workgroup shapes of the tiled kernels: query-stationary NQS x NKS,
// key-stationary NKB x NQS.  4 x 1 for both was best or within 3% of the
// best of nine shapes on MI355X for the c1 causal, c1 non-causal and c2
// causal backward; with stored probs, launch_tiled_probs also takes 4 x 2
// where the grid fills the device's slots better with it.
constexpr int kBwdQNqs = 4, kBwdQNks = 1, kBwdKvNkb = 4, kBwdKvNqs = 1;

hipError_t bwd_wait_expired(unsigned int* count, bool clear) { return wait_expired_take(count, clear); }

bool bwd_tiled_ok(const BwdArgs& a) {
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    return (a.D == 32 || a.D == 64) && a.ts % 4 == 0 && a.bs % 4 == 0 && a.hs % 4 == 0 && al(a.q) && al(a.k) &&
           al(a.v) && al(a.go) && al(a.dq) && al(a.dk) && al(a.dv) && al(a.probs) && al(a.o) &&
           ((int64_t)(a.S + 64) * a.ts + a.D) * 4 < ((int64_t)1 << 31);
}

// The one-workgroup-per-(b, h) kernels run a (b, h)'s steps in sequence, so
// one (b, h) takes 30-80 us whatever the batch.  With causal stored probs (and
// the D = 32 drop-in) they still beat the query-/key-stationary pair at any
// batch; rebuilding P from lse, and the D = 64 drop-in, only once the (b, h)
// pairs fill the CUs (S = 256, H = 8, B = 4: D = 64 from lse 83.2 -> 48.0 us,
// D = 32 from lse 32.3 -> 27.5 us, D = 64 drop-in 84.4 -> 77.8 us with the
// pair; B = 32 keeps the per-(b, h) kernels).
static bool bh_enough(const BwdArgs& a) {
    if (a.probs && (a.causal || a.D == 32)) return true;
    return (int64_t)a.B * a.H >= device_cus();
}

// The head-dim-split kernels of bwd_wide.h: D % 4 == 0 up to 256, 16-byte
// aligned rows; stored probs, or recompute mode from O and lse.
static bool bwd_wide_ok(const BwdArgs& a) {
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    const bool src = a.probs ? al(a.probs) : (a.o && a.lse && al(a.o));
    return src && a.D % 4 == 0 && a.D <= 256 && a.ts % 4 == 0 && a.bs % 4 == 0 && a.hs % 4 == 0 && al(a.q) &&
           al(a.k) && al(a.v) && al(a.go) && al(a.dq) && al(a.dk) && al(a.dv) &&
           ((int64_t)(a.S + 64) * a.ts + a.D) * 4 < ((int64_t)1 << 31);
}

bool bwd_recompute_ok(const BwdArgs& a) { return a.o && a.lse && (bwd_tiled_ok(a) || bwd_wide_ok(a)); }

bool bwd_uses_workspace(const BwdArgs& a) {
    if (!a.probs) return !bwd_tiled_ok(a);  // recompute mode: the wide kernels pass Dq through it
    return !(bwd_tiled_ok(a) && bh_enough(a) && (bwd::bh_ok(a) || bwd::bh_probs64_ok(a)));
}

hipError_t launch_attn_bwd(const BwdArgs& a, hipStream_t s) {
    // recompute mode (no probs): the tiled kernels, or the wide ones with the Dq workspace
    if (!a.probs && !(bwd_recompute_ok(a) && (bwd_tiled_ok(a) || a.dvec))) return hipErrorInvalidValue;
    if (bwd_tiled_ok(a)) {
        if (bh_enough(a) && bwd::bh_ok(a)) return bwd::launch_bh(a, s);
        if (bh_enough(a) && (bwd::bh_probs64_ok(a) || bwd::bh_lse64_ok(a))) return bwd::launch_bh64(a, s);
        if (a.probs) return a.D == 32 ? bwd::launch_tiled_probs<32>(a, s) : bwd::launch_tiled_probs<64>(a, s);
        if (a.D == 32)
            return bwd::launch_tiled<32, kBwdQNqs, kBwdQNks, kBwdKvNkb, kBwdKvNqs>(a, s);
        return bwd::launch_tiled<64, kBwdQNqs, kBwdQNks, kBwdKvNkb, kBwdKvNqs>(a, s);
    }
    if (bwd_wide_ok(a)) {
        if (a.D <= 32) return bwd::launch_wide<32, 4, 1, 2>(a, s);
        if (a.D <= 64) return bwd::launch_wide<64, 4, 1, 2>(a, s);
        if (a.D <= 128) return bwd::launch_wide<128, 4, 2, 2>(a, s);
        return bwd::launch_wide<256, 2, 4, 1>(a, s);
    }
    if (a.D <= 32) return launch_dp<32>(a, s);
    if (a.D <= 64) return launch_dp<64>(a, s);
    if (a.D <= 128) return launch_dp<128>(a, s);
    const int64_t blocks = ((int64_t)a.B * a.H * a.S + 255) / 256;
    if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(bwd_generic_q_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(bwd_generic_kv_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace hipgpt
