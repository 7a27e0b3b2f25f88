// helpers.hip -- HipGPT's unfused single-head attention helpers.
//
// Replaces scaled_dot_product_kernel, softmax_kernel and
// attention_weighted_sum_kernel (HipGPT src/hip_kernels.cpp:454-532, declared
// include/hip_kernels.h:44-46).  HipGPT itself no longer calls them (the
// flash path replaced them), but they are part of the header a drop-in must
// provide.  Layouts: Q, K, V, O are [B*S][D]; scores / probs are [B*S][S];
// non-causal.
//
// All three stream the [B*S][S] matrix through HBM once: written by the
// scores, read and written by the softmax, read by the weighted sum.
//   * scores = Q K^T * rsqrt(D): a workgroup owns 4 query tiles of 32 rows
//     of one sequence (Q in registers, one tile per wave) and streams a range
//     of key tiles through LDS (double-buffered, one barrier per tile), so
//     each K tile is read once per 128 queries.  S = Q K^T on
//     v_mfma_f32_32x32x2_f32 with A = Q, B = K^T; each wave transposes its
//     32x32 result through LDS and writes it as 16-byte non-temporal stores
//     (8 full 128-byte row segments per instruction).  Sequences with few
//     query tiles split their keys over several workgroups (no reduction
//     needed: every score is written once).
//   * row softmax: a row held in registers (float4 per lane, up to 2048
//     columns), read once and written once; longer or unaligned rows use
//     three read sweeps and one write.
//   * out = P V: a workgroup owns 4 query tiles of one sequence; V tiles are
//     staged through LDS once per 128 queries; each lane reads 16
//     consecutive probabilities of its query as four float4 (A operand, two
//     tiles ahead) and V^T from LDS (B operand).  Problems with fewer than 256
//     such workgroups instead split one query tile's keys over 4 waves and
//     add the partial O tiles in LDS.
// Head dims other than 32/64/128, unaligned pointers and (weighted sum) S not
// a multiple of 4 use the per-element kernels at the end of the file.
// Workgroup numbers go through xcd_remap so the workgroups of one sequence
// share an L2.
#include "common.h"
#include "fa_common.h"
#include "kernels.h"

namespace hipgpt {

// Weighted-sum output stores: whole 128-byte row segments per half-wave,
// written non-temporally (a8: 21.6 -> 20.1 us against plain stores).
__device__ __forceinline__ void nt_store(float* p, float v) { __builtin_nontemporal_store(v, p); }

namespace {

using fa::acc_key;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Scores: target workgroup count before keys are split (2 per CU), and the
// fewest key tiles a split keeps.
constexpr int kSdpTargetGroups = 512;
constexpr int kSdpMinSplitTiles = 2;
// Weighted sum: fewest query-group workgroups for the grouped kernel.
constexpr int kWsumMinGroups = 256;

// ---------------------------------------------------------------- Q K^T
// Workgroup (sequence b, query group qg, key chunk kc); wave w owns query
// tile qg*4 + w: lane (c, hf) holds Q[q0 + c][hf*DP/2 + s] (A operand) and
// reads K[k0 + c][hf*DP/2 + s] from LDS (B operand), so accumulator register
// r is scores[q0 + acc_key(r, hf)][k0 + c].
template <int DP>
__global__ __launch_bounds__(256) void sdp_tiles_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                                                        float* __restrict__ scores, int S, float inv, int n_qg,
                                                        int n_kc, int kc_tiles, int vec_store) {
    constexpr int KP = DP + 4;   // K row pitch: conflict-free ds_read_b128 rows
    constexpr int NF = DP / 8;   // float4 operand pieces per lane
    constexpr int NL = DP / 32;  // float4 per thread per staged K tile
    constexpr int TP = 36;       // transpose tile pitch
    __shared__ float ks[2][32 * KP];
    __shared__ float tr[4][32 * TP];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 31, hf = lane >> 5;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int kc = lid % n_kc, t = lid / n_kc, qg = t % n_qg, b = t / n_qg;
    const int q0 = (qg * 4 + wave) * 32;
    const int nt = (S + 31) / 32;
    const int kt0 = kc * kc_tiles, kt1 = min(nt, kt0 + kc_tiles);
    const float* Kb = K + (int64_t)b * S * DP;
    float* out = scores + (int64_t)b * S * S;

    floatx4 qf[NF];
    {
        const bool ok = q0 + c < S;
        const float* p = Q + ((int64_t)b * S + (ok ? q0 + c : 0)) * DP + hf * (DP / 2);
#pragma unroll
        for (int i = 0; i < NF; ++i)
            qf[i] = ok ? *reinterpret_cast<const floatx4*>(p + 4 * i) : floatx4{0.f, 0.f, 0.f, 0.f};
    }
    floatx4 kr[NL];
    auto load_k = [&](int kt) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int idx = threadIdx.x + 256 * i, row = idx / (DP / 4), c4 = idx % (DP / 4);
            const int key = kt * 32 + row;
            kr[i] = key < S ? *reinterpret_cast<const floatx4*>(Kb + (int64_t)key * DP + c4 * 4)
                            : floatx4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto store_k = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int idx = threadIdx.x + 256 * i, row = idx / (DP / 4), c4 = idx % (DP / 4);
            *reinterpret_cast<floatx4*>(&ks[buf][row * KP + c4 * 4]) = kr[i];
        }
    };

    if (kt0 < kt1) {
        load_k(kt0);
        store_k(0);
    }
    __syncthreads();
    const bool active = q0 < S;  // the last group's spare waves only stage K
    for (int kt = kt0; kt < kt1; ++kt) {
        const int buf = (kt - kt0) & 1;
        if (kt + 1 < kt1) load_k(kt + 1);
        if (active) {
            const float* kp = &ks[buf][c * KP + hf * (DP / 2)];
            floatx4 kf[NF];
#pragma unroll
            for (int i = 0; i < NF; ++i) kf[i] = *reinterpret_cast<const floatx4*>(kp + 4 * i);
            floatx16 acc;
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
            for (int i = 0; i < NF; ++i)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(qf[i][u], kf[i][u], acc, 0, 0, 0);
            // Transpose through this wave's LDS tile: lane l then holds row
            // 8i + l/8, columns 4(l%8)..+3.  A wave's LDS accesses complete in
            // order, so no barrier is needed between the writes and reads.
            float* tw = tr[wave];
#pragma unroll
            for (int r = 0; r < 16; ++r) tw[acc_key(r, hf) * TP + c] = acc[r] * inv;
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = i * 8 + (lane >> 3), col = (lane & 7) * 4;
                const floatx4 v = *reinterpret_cast<const floatx4*>(tw + row * TP + col);
                const int q = q0 + row, key = kt * 32 + col;
                if (q < S) {
                    float* dst = out + (int64_t)q * S + key;
                    if (vec_store && key < S) {  // S % 4 == 0: key < S covers the whole float4
                        __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(dst));
                    } else {
#pragma unroll
                        for (int u = 0; u < 4; ++u)
                            if (key + u < S) dst[u] = v[u];
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
        if (kt + 1 < kt1) store_k(buf ^ 1);
        __syncthreads();
    }
}

// ---------------------------------------------------------------- softmax
// One wave per row, the row in registers: lane l holds columns
// 4*(l + 64*i) .. +3, i < NV.  Padding lanes read -inf (exp2 -> 0).
template <int NV>
__global__ __launch_bounds__(256) void softmax_vec_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                          int64_t rows, int S) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const floatx4* x = reinterpret_cast<const floatx4*>(in + row * S);
    floatx4* y = reinterpret_cast<floatx4*>(out + row * S);
    const int n4 = S / 4;
    floatx4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = lane + 64 * i;
        v[i] = j < n4 ? x[j] : floatx4{kNegInf, kNegInf, kNegInf, kNegInf};
    }
    float m = kMaxInit;
#pragma unroll
    for (int i = 0; i < NV; ++i) m = fmaxf(fmaxf(fmaxf(m, v[i][0]), fmaxf(v[i][1], v[i][2])), v[i][3]);
    m = wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            v[i][u] = fast_exp2((v[i][u] - m) * kLog2e);
            s += v[i][u];
        }
    const float inv = 1.0f / fmaxf(wave_sum(s), 1e-20f);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = lane + 64 * i;
        if (j < n4) y[j] = v[i] * inv;  // plain: non-temporal measured 24.0 -> 24.6 us at a8
    }
}

// Any S and alignment: max sweep, sum sweep, write sweep (the row is read
// three times, from L2 after the first, and written once).
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                           int64_t rows, int S) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* x = in + row * S;
    float* y = out + row * S;
    float m = kMaxInit;
    for (int j = lane; j < S; j += 64) m = fmaxf(m, x[j]);
    m = wave_max(m);
    float s = 0.f;
    for (int j = lane; j < S; j += 64) s += fast_exp2((x[j] - m) * kLog2e);
    const float inv = 1.0f / fmaxf(wave_sum(s), 1e-20f);
    for (int j = lane; j < S; j += 64) y[j] = fast_exp2((x[j] - m) * kLog2e) * inv;
}

// ---------------------------------------------------------------- P V
// MFMA step s of a key tile contracts key hf*16 + s for lane half hf: lane
// (c, hf) reads P[q][k0 + hf*16 .. +16) as four float4 (A operand) and
// V[k0 + hf*16 + s][db*32 + c] (B operand); accumulator block db, register r
// is O[q0 + acc_key(r, hf)][db*32 + c].  S % 4 == 0, so a float4 of P is
// either all inside the row or all past its end.
template <int DP>
struct WsumTile {
    static constexpr int NB = DP / 32;
    __device__ __forceinline__ static void load_p(floatx4 (&pf)[4], const float* prow, bool qok, int kt, int hf,
                                                  int S) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int key = kt * 32 + hf * 16 + 4 * g;
            pf[g] = (qok && key < S) ? *reinterpret_cast<const floatx4*>(prow + kt * 32 + 4 * g)
                                     : floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
};

// P of the weighted sum goes through a per-wave LDS transpose, whole 128-byte
// rows per load, instead of straight in the MFMA operand layout (32 bytes of
// each of 32 rows per load): a8, cache-rotated, 20.1 -> 19.6 us (mean of
// four).  Deeper P prefetch (3 or 4 tiles in flight instead of 2) measured
// slower either way, and so did requesting V of the next tile before P.

// Workgroup (sequence b, query group qg); wave w owns query tile qg*4 + w
// over all keys; V tiles staged through LDS (double-buffered, one barrier per
// tile); P two tiles ahead in registers.
template <int DP>
__global__ __launch_bounds__(256) void wsum_tiles_kernel(const float* __restrict__ P, const float* __restrict__ V,
                                                         float* __restrict__ O, int S, int n_qg) {
    constexpr int NB = DP / 32;
    constexpr int NL = DP / 32;  // float4 per thread per staged V tile
    __shared__ float vs[2][32 * DP];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 31, hf = lane >> 5;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int qg = lid % n_qg, b = lid / n_qg;
    const int q0 = (qg * 4 + wave) * 32;
    const int nt = (S + 31) / 32;
    const float* Vb = V + (int64_t)b * S * DP;

    floatx4 vr[NL];
    auto load_v = [&](int kt) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int idx = threadIdx.x + 256 * i, row = idx / (DP / 4), c4 = idx % (DP / 4);
            const int key = kt * 32 + row;
            vr[i] = key < S ? *reinterpret_cast<const floatx4*>(Vb + (int64_t)key * DP + c4 * 4)
                            : floatx4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto store_v = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int idx = threadIdx.x + 256 * i, row = idx / (DP / 4), c4 = idx % (DP / 4);
            *reinterpret_cast<floatx4*>(&vs[buf][row * DP + c4 * 4]) = vr[i];
        }
    };

    floatx16 acc[NB];
#pragma unroll
    for (int db = 0; db < NB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    // P through a per-wave LDS transpose: each load instruction reads 8 whole
    // 128-byte rows of the tile (lane: row rr + 8i, keys cc .. cc+3), and the
    // MFMA operands (lane: query c, keys 16hf .. 16hf+15) are read back from
    // the 32 x 36 scratch (the pitch puts 16 lanes' rows on disjoint banks).
    __shared__ __attribute__((aligned(16))) float px[4][32 * 36];
    float* const X = px[wave];
    const int rr = lane >> 3, cc = 4 * (lane & 7);
    const float* ptile = P + ((int64_t)b * S + q0) * S;
    auto load_tile = [&](floatx4 (&pf)[4], int kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 8 * i + rr, key = kt * 32 + cc;
            pf[i] = (q0 + row < S && key < S) ? *reinterpret_cast<const floatx4*>(ptile + (int64_t)row * S + key)
                                              : floatx4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto operands = [&](const floatx4 (&pf)[4], floatx4 (&op)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<floatx4*>(X + (8 * i + rr) * 36 + cc) = pf[i];
        asm volatile("" ::: "memory");  // other lanes' writes (the wave's LDS accesses are in order)
#pragma unroll
        for (int g = 0; g < 4; ++g) op[g] = *reinterpret_cast<const floatx4*>(X + c * 36 + 16 * hf + 4 * g);
        asm volatile("" ::: "memory");  // the next tile's writes come after these reads
    };
    floatx4 pa[4], pb[4];  // P of tiles kt and kt + 1
    load_tile(pa, 0);
    if (1 < nt) load_tile(pb, 1);
    load_v(0);
    store_v(0);
    __syncthreads();
    for (int kt = 0; kt < nt; ++kt) {
        const int buf = kt & 1;
        floatx4 cur[4];
        operands(pa, cur);
#pragma unroll
        for (int g = 0; g < 4; ++g) pa[g] = pb[g];
        if (kt + 2 < nt) load_tile(pb, kt + 2);
        if (kt + 1 < nt) load_v(kt + 1);
        const float* vp = &vs[buf][(hf * 16) * DP + c];
#pragma unroll
        for (int db = 0; db < NB; ++db)
#pragma unroll
            for (int s = 0; s < 16; ++s)
                acc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[s >> 2][s & 3], vp[s * DP + db * 32], acc[db], 0, 0,
                                                               0);
        if (kt + 1 < nt) store_v(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int db = 0; db < NB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int q = q0 + acc_key(r, hf);
            if (q < S) nt_store(&O[((int64_t)b * S + q) * DP + db * 32 + c], acc[db][r]);
        }
}

// Few query groups: workgroup (sequence b, query tile); wave w takes key
// tiles w, w+4, ... with V read straight from global memory, and the four
// partial O tiles are added in LDS.
template <int DP>
__global__ __launch_bounds__(256) void wsum_split_kernel(const float* __restrict__ P, const float* __restrict__ V,
                                                         float* __restrict__ O, int S) {
    constexpr int NB = DP / 32;
    using T = WsumTile<DP>;
    __shared__ float red[4][NB][16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 31, hf = lane >> 5;
    const int nt = (S + 31) / 32;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int q0 = (lid % nt) * 32, b = lid / nt;
    const bool qok = q0 + c < S;
    const float* prow = P + ((int64_t)b * S + (qok ? q0 + c : 0)) * S + hf * 16;
    const float* Vb = V + (int64_t)b * S * DP + (int64_t)(hf * 16) * DP + c;

    floatx16 acc[NB];
#pragma unroll
    for (int db = 0; db < NB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;

    floatx4 pf[4];
    int kt = wave;
    if (kt < nt) T::load_p(pf, prow, qok, kt, hf, S);
    for (; kt < nt; kt += 4) {
        floatx4 cur[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) cur[g] = pf[g];
        if (kt + 4 < nt) T::load_p(pf, prow, qok, kt + 4, hf, S);
        const float* vp = Vb + (int64_t)(kt * 32) * DP;
        const int kbase = kt * 32 + hf * 16;
#pragma unroll
        for (int db = 0; db < NB; ++db) {
            float vv[16];
#pragma unroll
            for (int s = 0; s < 16; ++s) vv[s] = kbase + s < S ? vp[s * DP + db * 32] : 0.f;
#pragma unroll
            for (int s = 0; s < 16; ++s)
                acc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[s >> 2][s & 3], vv[s], acc[db], 0, 0, 0);
        }
    }

#pragma unroll
    for (int db = 0; db < NB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave][db][r][lane] = acc[db][r];
    __syncthreads();
    // Thread t adds element (db, r, lane) = t + 256*i of the four partials and
    // stores it: consecutive threads write consecutive columns of a row.
#pragma unroll
    for (int i = 0; i < NB * 4; ++i) {
        const int e = threadIdx.x + 256 * i;
        const int l = e & 63, r = (e >> 6) & 15, db = e >> 10;
        const float sum = red[0][db][r][l] + red[1][db][r][l] + red[2][db][r][l] + red[3][db][r][l];
        const int q = q0 + acc_key(r, l >> 5);
        if (q < S) nt_store(&O[((int64_t)b * S + q) * DP + db * 32 + (l & 31)], sum);
    }
}

// ---------------------------------------------------------------- any D
// Per-element kernels for head dims other than 32/64/128, unaligned
// pointers, and (weighted sum) S not a multiple of 4.
__global__ __launch_bounds__(256) void sdp_scalar_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                                                         float* __restrict__ scores, int B, int S, int D, float inv) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = (int64_t)B * S * S;
    if (idx >= n) return;
    const int64_t tok = idx / S;
    const int j = (int)(idx % S);
    const float* q = Q + tok * D;
    const float* k = K + ((tok / S) * S + j) * (int64_t)D;
    float acc = 0.f;
    for (int d = 0; d < D; ++d) acc = fmaf(q[d], k[d], acc);
    scores[idx] = acc * inv;
}

__global__ __launch_bounds__(256) void wsum_scalar_kernel(const float* __restrict__ P, const float* __restrict__ V,
                                                          float* __restrict__ O, int B, int S, int D) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = (int64_t)B * S * D;
    if (idx >= n) return;
    const int64_t tok = idx / D;
    const int d = (int)(idx % D);
    const float* p = P + tok * S;
    const float* v = V + (tok / S) * S * (int64_t)D + d;
    float acc = 0.f;
    for (int j = 0; j < S; ++j) acc = fmaf(p[j], v[(int64_t)j * D], acc);
    O[idx] = acc;
}

hipError_t grid_1d(int64_t n, unsigned& blocks) {
    if (n > 0x7fffffff) return hipErrorInvalidConfiguration;
    blocks = (unsigned)n;
    return hipSuccess;
}

template <int DP>
void launch_sdp_tiles(const float* Q, const float* K, float* scores, int S, float inv, hipStream_t s,
                      unsigned blocks, int n_qg, int n_kc, int kc_tiles, int vec_store) {
    hipLaunchKernelGGL(sdp_tiles_kernel<DP>, dim3(blocks), dim3(256), 0, s, Q, K, scores, S, inv, n_qg, n_kc, kc_tiles,
                       vec_store);
}

template <int DP>
void launch_wsum_dp(const float* P, const float* V, float* O, int B, int S, hipStream_t s) {
    const int nt = (S + 31) / 32, n_qg = (nt + 3) / 4;
    if ((int64_t)B * n_qg >= kWsumMinGroups)
        hipLaunchKernelGGL(wsum_tiles_kernel<DP>, dim3((unsigned)((int64_t)B * n_qg)), dim3(256), 0, s, P, V, O, S,
                           n_qg);
    else
        hipLaunchKernelGGL(wsum_split_kernel<DP>, dim3((unsigned)((int64_t)B * nt)), dim3(256), 0, s, P, V, O, S);
}

}  // namespace

hipError_t launch_sdp(const float* Q, const float* K, float* scores, int B, int S, int D, hipStream_t s) {
    const float inv = 1.0f / sqrtf((float)D);
    if ((D == 32 || D == 64 || D == 128) && aligned16(Q) && aligned16(K)) {
        const int nt = (S + 31) / 32, n_qg = (nt + 3) / 4;
        int n_kc = 1;
        while ((int64_t)B * n_qg * n_kc < kSdpTargetGroups && nt / (2 * n_kc) >= kSdpMinSplitTiles) n_kc *= 2;
        const int kc_tiles = (nt + n_kc - 1) / n_kc;
        const int vec_store = (S % 4 == 0) && aligned16(scores);
        unsigned blocks;
        const hipError_t e = grid_1d((int64_t)B * n_qg * n_kc, blocks);
        if (e != hipSuccess) return e;
        if (D == 32) launch_sdp_tiles<32>(Q, K, scores, S, inv, s, blocks, n_qg, n_kc, kc_tiles, vec_store);
        if (D == 64) launch_sdp_tiles<64>(Q, K, scores, S, inv, s, blocks, n_qg, n_kc, kc_tiles, vec_store);
        if (D == 128) launch_sdp_tiles<128>(Q, K, scores, S, inv, s, blocks, n_qg, n_kc, kc_tiles, vec_store);
        return hipGetLastError();
    }
    unsigned blocks;
    const hipError_t e = grid_1d(((int64_t)B * S * S + 255) / 256, blocks);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(sdp_scalar_kernel, dim3(blocks), dim3(256), 0, s, Q, K, scores, B, S, D, inv);
    return hipGetLastError();
}

hipError_t launch_softmax_rows(const float* in, float* out, int B, int S, hipStream_t s) {
    const int64_t rows = (int64_t)B * S;
    unsigned blocks;
    const hipError_t e = grid_1d((rows + 3) / 4, blocks);
    if (e != hipSuccess) return e;
    const dim3 grid(blocks);
    if (S % 4 == 0 && aligned16(in) && aligned16(out) && S <= 2048) {
        if (S <= 256) hipLaunchKernelGGL(softmax_vec_kernel<1>, grid, dim3(256), 0, s, in, out, rows, S);
        else if (S <= 512) hipLaunchKernelGGL(softmax_vec_kernel<2>, grid, dim3(256), 0, s, in, out, rows, S);
        else if (S <= 1024) hipLaunchKernelGGL(softmax_vec_kernel<4>, grid, dim3(256), 0, s, in, out, rows, S);
        else hipLaunchKernelGGL(softmax_vec_kernel<8>, grid, dim3(256), 0, s, in, out, rows, S);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(softmax_rows_kernel, grid, dim3(256), 0, s, in, out, rows, S);
    return hipGetLastError();
}

hipError_t launch_wsum(const float* P, const float* V, float* O, int B, int S, int D, hipStream_t s) {
    if ((D == 32 || D == 64 || D == 128) && S % 4 == 0 && aligned16(P) && aligned16(V) && aligned16(O)) {
        if ((int64_t)B * ((S + 31) / 32) > 0x7fffffff) return hipErrorInvalidConfiguration;
        if (D == 32) launch_wsum_dp<32>(P, V, O, B, S, s);
        if (D == 64) launch_wsum_dp<64>(P, V, O, B, S, s);
        if (D == 128) launch_wsum_dp<128>(P, V, O, B, S, s);
        return hipGetLastError();
    }
    unsigned blocks;
    const hipError_t e = grid_1d(((int64_t)B * S * D + 255) / 256, blocks);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(wsum_scalar_kernel, dim3(blocks), dim3(256), 0, s, P, V, O, B, S, D);
    return hipGetLastError();
}

}  // namespace hipgpt
