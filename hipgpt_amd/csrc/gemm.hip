// gemm.hip -- fp32 GEMM + bias on gfx950 MFMA: the projections either side
// of the attention (QKV projection and output projection).
//
// Replaces matmul_add_bias_tiled_kernel / launch_matmul_add_bias and
// matmul_tiled_kernel / launch_matmul (HipGPT src/hip_kernels.cpp:113-154,
// :70-109), called from TransformerLayer::self_attention_forward
// (src/transformer_layer.cpp:217, :220):
//     C[m][n] = sum_k A[m][k] W[k][n] (+ bias[n])
// with A [M][K] (row stride lda), W [K][N] (row stride ldw).  Output column
// n goes to C + (n / seg_w) * seg_stride + m * ldc + n % seg_w, which is the
// plain row-major [M][N] buffer for seg_w = N and, for the QKV projection
// (N = 3E, seg_w = E, seg_stride = M*E), the planar [Q|K|V] buffer the
// attention launcher reads.  Output fp32 or bf16 (RNE).
//
// Tiling: a workgroup owns a BM x BN tile of C and walks K in steps of GBK.
// Each wave computes a WM x WN sub-tile as C^T = W^T A^T on
// v_mfma_f32_32x32x2_f32, so an accumulator register group holds four
// consecutive output columns of one row (16-byte stores, 16-byte bias loads).
// Operand staging: global -> registers -> LDS, double buffered, one barrier
// per k-tile; the next tile's global loads are in flight during the MFMAs.
//   A tile [BM][GBK] (pitch GBK+4 floats): lane (c, h) reads row c,
//     k = (GBK/2)h + s as ds_read_b128 (four k-steps per read).
//   W tile [GBK][BN] (pitch BN+4, second half of the k rows shifted by 32
//     floats so the two lane halves read different banks): lane (c, h) reads
//     W[(GBK/2)h + s][c] as one dword per k-step.
// MFMA 32x32x2 f32 operand layout (lane l, c = l & 31, h = l >> 5): A-operand
// value = row c of the MFMA's M dim, B-operand value = column c of its N dim,
// both at contraction index h of the step; here contraction index
// k = (GBK/2)h + s at step s, the same bijection for both operands.
#include "common.h"
#include "kernels.h"

namespace hipgpt {

namespace {

template <int BM, int BN, int WM, int WN, int GBK_ = 32>
struct Cfg {
    static constexpr int GBK = GBK_;         // k per tile
    static constexpr int APITCH = GBK + 4;   // A tile row pitch, floats
    static constexpr int ACPR = GBK / 4;     // 16-byte chunks per A tile row
    static constexpr int WAVES_M = BM / WM;
    static constexpr int WAVES_N = BN / WN;
    static constexpr int NW = WAVES_M * WAVES_N;
    static constexpr int NT = NW * 64;
    static constexpr int MB = WM / 32;  // m blocks per wave (MFMA N dim)
    static constexpr int NB = WN / 32;  // n blocks per wave (MFMA M dim)
    static constexpr int WPITCH = BN + 4;
    static constexpr int A_ELEMS = BM * APITCH;
    static constexpr int W_ELEMS = GBK * WPITCH + 32;
    static constexpr int STAGE = A_ELEMS + W_ELEMS;
    static constexpr int A_CHUNKS = BM * GBK / 4;
    static constexpr int W_CHUNKS = GBK * BN / 4;
    static constexpr int A_PER = A_CHUNKS / NT;
    static constexpr int W_PER = W_CHUNKS / NT;
    static_assert(A_CHUNKS % NT == 0 && W_CHUNKS % NT == 0, "tile loads must split evenly over the workgroup");
    static_assert(WM % 32 == 0 && WN % 32 == 0 && BM % WM == 0 && BN % WN == 0, "bad tile shape");
    // W row r of the tile lives at r * WPITCH + (r >= GBK/2 ? 32 : 0).
    __device__ __forceinline__ static int wrow(int r) { return r * WPITCH + (r >= GBK / 2 ? 32 : 0); }
};

__device__ __forceinline__ floatx4 zero4() { return floatx4{0.f, 0.f, 0.f, 0.f}; }

// KF: K is a multiple of GBK (16-byte path only), so no k-tile runs past K:
// the k offset of the loads rides in the buffer instruction's scalar offset
// and the per-element k mask goes away.  With the k loop unrolled by two
// (UNROLL2: each stage buffer at a constant address, the operand reads at
// loop-invariant bases) the loop issues no VALU work beyond a loop test,
// which matters because fp32 VALU ops take MFMA issue cycles on gfx950.
// Cache-rotated, us: c1 QKV 32.6 -> 30.6, c1 out 14.9 -> 13.7, c3 QKV
// 246 -> 232, c3 out 85.2 -> 80.1 (KF alone: c3 QKV 244, c1 level).
template <int BM, int BN, int WM, int WN, int GBK, int NACC, bool VEC, bool BF16OUT, bool KF>
__global__ __launch_bounds__(BM / WM * (BN / WN) * 64) void gemm_bias_kernel(GemmArgs g) {
    using C = Cfg<BM, BN, WM, WN, GBK>;
    constexpr int APITCH = C::APITCH;
    constexpr int ACPR = C::ACPR;
    constexpr int HS = GBK / 2;  // k-steps per tile (each step takes k = HS*h + s)
    __shared__ __attribute__((aligned(16))) float lds[2 * C::STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int c = lane & 31, h = lane >> 5;
    const int tiles_n = (g.N + BN - 1) / BN;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int wm0 = (wave / C::WAVES_N) * WM;  // wave's rows within the tile
    const int wn0 = (wave % C::WAVES_N) * WN;  // wave's columns within the tile
    const int K = g.K;
    const int nkt = (K + GBK - 1) / GBK;

    // ---- global -> register staging of one k-tile ----
    floatx4 ar[C::A_PER], wr[C::W_PER];
    __amdgpu_buffer_rsrc_t ars, wrs;
    int aoff[C::A_PER], woff[C::W_PER];
    if constexpr (VEC) {
        const int rows = min(BM, g.M - m0);
        const int cols = min(BN, g.N - n0);
        ars = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.A + (int64_t)m0 * g.lda), 0,
                                                (int)(((int64_t)(rows - 1) * g.lda + K) * 4), kBufferFlags);
        wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.W + n0), 0,
                                                (int)(((int64_t)(K - 1) * g.ldw + cols) * 4), kBufferFlags);
#pragma unroll
        for (int i = 0; i < C::A_PER; ++i) {
            const int f = tid + i * C::NT;
            aoff[i] = (int)(((f / ACPR) * g.lda + (f % ACPR) * 4) * 4);
        }
#pragma unroll
        for (int i = 0; i < C::W_PER; ++i) {
            const int f = tid + i * C::NT;
            const int kr = f / (BN / 4), nc = (f % (BN / 4)) * 4;
            // KF: columns past N re-read column n0 (in bounds; they only feed
            // outputs that are never stored), as the scalar k offset is outside
            // the buffer's range check
            woff[i] = (int)((kr * g.ldw + (KF && nc >= cols ? 0 : nc)) * 4);
        }
    }
    auto load = [&](int kt) {
        const int k0 = kt * GBK;
#pragma unroll
        for (int i = 0; i < C::A_PER; ++i) {
            const int f = tid + i * C::NT;
            const int r = f / ACPR, kc = (f % ACPR) * 4;
            if constexpr (VEC && KF) {
                // rows past M read as zero (their voffset is past the range)
                ar[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(ars, aoff[i], k0 * 4, 0));
            } else if constexpr (VEC) {
                // rows past M read as zero (buffer range); k past K is masked
                // here because it would read the next row's values
                const floatx4 v = __builtin_bit_cast(
                    floatx4, __builtin_amdgcn_raw_buffer_load_b128(ars, aoff[i] + k0 * 4, 0, 0));
                ar[i] = (k0 + kc < K) ? v : zero4();
            } else {
                const int m = m0 + r;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int k = k0 + kc + j;
                    ar[i][j] = (m < g.M && k < K) ? g.A[(int64_t)m * g.lda + k] : 0.f;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < C::W_PER; ++i) {
            const int f = tid + i * C::NT;
            const int kr = f / (BN / 4), nc = (f % (BN / 4)) * 4;
            if constexpr (VEC && KF) {
                wr[i] = __builtin_bit_cast(
                    floatx4, __builtin_amdgcn_raw_buffer_load_b128(wrs, woff[i], (int)((int64_t)k0 * g.ldw * 4), 0));
            } else if constexpr (VEC) {
                // rows past K read as zero; columns past N only feed outputs
                // that are never stored
                wr[i] = __builtin_bit_cast(
                    floatx4, __builtin_amdgcn_raw_buffer_load_b128(wrs, woff[i] + (int)((int64_t)k0 * g.ldw * 4), 0, 0));
            } else {
                const int k = k0 + kr;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int n = n0 + nc + j;
                    wr[i][j] = (k < K && n < g.N) ? g.W[(int64_t)k * g.ldw + n] : 0.f;
                }
            }
        }
    };
    auto store = [&](float* st) {
#pragma unroll
        for (int i = 0; i < C::A_PER; ++i) {
            const int f = tid + i * C::NT;
            *reinterpret_cast<floatx4*>(st + (f / ACPR) * APITCH + (f % ACPR) * 4) = ar[i];
        }
        float* ws = st + C::A_ELEMS;
#pragma unroll
        for (int i = 0; i < C::W_PER; ++i) {
            const int f = tid + i * C::NT;
            *reinterpret_cast<floatx4*>(ws + C::wrow(f / (BN / 4)) + (f % (BN / 4)) * 4) = wr[i];
        }
    };

    // NACC independent accumulator chains per output block (k-steps
    // alternate between them), summed in the epilogue.
    floatx16 acc[NACC][C::NB][C::MB];
#pragma unroll
    for (int x = 0; x < NACC; ++x)
#pragma unroll
        for (int i = 0; i < C::NB; ++i)
#pragma unroll
            for (int j = 0; j < C::MB; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[x][i][j][r] = 0.f;

    auto compute = [&](const float* st) {
        const float* As = st + (wm0 + c) * APITCH + h * HS;
        const float* Ws = st + C::A_ELEMS + wn0 + c;
#pragma unroll
        for (int q = 0; q < HS / 4; ++q) {
            floatx4 av[C::MB];
#pragma unroll
            for (int j = 0; j < C::MB; ++j) av[j] = *reinterpret_cast<const floatx4*>(As + j * 32 * APITCH + 4 * q);
            float wv[C::NB][4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int row = C::wrow(h * HS + 4 * q + u);
#pragma unroll
                for (int i = 0; i < C::NB; ++i) wv[i][u] = Ws[row + 32 * i];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int i = 0; i < C::NB; ++i)
#pragma unroll
                    for (int j = 0; j < C::MB; ++j)
                        acc[u % NACC][i][j] =
                            __builtin_amdgcn_mfma_f32_32x32x2f32(wv[i][u], av[j][u], acc[u % NACC][i][j], 0, 0, 0);
        }
    };

    if (nkt > 0) {
        load(0);
        store(lds);
    }
    __syncthreads();
    // two k-tiles per iteration, so each stage buffer's address is a constant
    auto step = [&](int kt, auto stage_tag) {
        constexpr int SB = decltype(stage_tag)::value;
        if (kt + 1 < nkt) load(kt + 1);
        compute(lds + SB * C::STAGE);
        if (kt + 1 < nkt) store(lds + (1 - SB) * C::STAGE);
        __syncthreads();
    };
    for (int kt = 0; kt < nkt; kt += 2) {
        step(kt, std::integral_constant<int, 0>{});
        if (kt + 1 < nkt) step(kt + 1, std::integral_constant<int, 1>{});
    }

    // ---- epilogue, whole-row path: each 32 x 32 block (+ bias) goes through
    // a per-wave scratch in the (now idle) stage buffers and leaves as whole
    // 128-byte row segments, non-temporally, when the block is inside C, fp32,
    // and its 32 columns stay in one segment ----
    constexpr bool ROWS_T = VEC && !BF16OUT && C::NW * 32 * 36 <= 2 * C::STAGE;
    if constexpr (ROWS_T) {
        float* const X = lds + wave * 32 * 36;
        const int rr = lane >> 3, cc = 4 * (lane & 7);
#pragma unroll
        for (int i = 0; i < C::NB; ++i) {
            const int nb = n0 + wn0 + 32 * i;  // first column of the block
#pragma unroll
            for (int j = 0; j < C::MB; ++j) {
                const int mb = m0 + wm0 + 32 * j;  // first row of the block
                const bool whole = mb + 32 <= g.M && nb + 32 <= g.N && nb / g.seg_w == (nb + 31) / g.seg_w;
                if (!whole) continue;  // left to the general path below
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int n = nb + 8 * q + 4 * h;
                    const floatx4 bv = g.bias ? *reinterpret_cast<const floatx4*>(g.bias + n) : zero4();
                    floatx4 v;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        float t = acc[0][i][j][4 * q + u];
#pragma unroll
                        for (int x = 1; x < NACC; ++x) t += acc[x][i][j][4 * q + u];
                        v[u] = t + bv[u];
                    }
                    *reinterpret_cast<floatx4*>(X + c * 36 + 8 * q + 4 * h) = v;
                }
                asm volatile("" ::: "memory");  // other lanes' writes (the wave's LDS accesses are in order)
                float* const cb = static_cast<float*>(g.C) + (int64_t)(nb / g.seg_w) * g.seg_stride + nb % g.seg_w;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int row = 8 * k + rr;
                    const floatx4 v = *reinterpret_cast<const floatx4*>(X + row * 36 + cc);
                    __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(cb + (int64_t)(mb + row) * g.ldc + cc));
                }
                asm volatile("" ::: "memory");  // the next block's writes come after these reads
            }
        }
    }

    // ---- epilogue: + bias, store (register group q -> columns 8q + 4h .. +3) ----
#pragma unroll
    for (int i = 0; i < C::NB; ++i) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = n0 + wn0 + 32 * i + 8 * q + 4 * h;
            floatx4 bv = zero4();
            if (g.bias) {
                if (VEC) {
                    if (n < g.N) bv = *reinterpret_cast<const floatx4*>(g.bias + n);
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u) bv[u] = (n + u < g.N) ? g.bias[n + u] : 0.f;
                }
            }
#pragma unroll
            for (int j = 0; j < C::MB; ++j) {
                const int m = m0 + wm0 + 32 * j + c;
                if (m >= g.M) continue;
                if constexpr (ROWS_T) {  // stored above
                    const int mb = m0 + wm0 + 32 * j, nb = n0 + wn0 + 32 * i;
                    if (mb + 32 <= g.M && nb + 32 <= g.N && nb / g.seg_w == (nb + 31) / g.seg_w) continue;
                }
                floatx4 v;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    float t = acc[0][i][j][4 * q + u];
#pragma unroll
                    for (int x = 1; x < NACC; ++x) t += acc[x][i][j][4 * q + u];
                    v[u] = t + bv[u];
                }
                if (VEC) {
                    if (n >= g.N) continue;
                    const int64_t off = (int64_t)(n / g.seg_w) * g.seg_stride + (int64_t)m * g.ldc + n % g.seg_w;
                    if (BF16OUT) {
                        bf16x4 o;
#pragma unroll
                        for (int u = 0; u < 4; ++u) o[u] = (__bf16)v[u];
                        *reinterpret_cast<bf16x4*>(static_cast<__bf16*>(g.C) + off) = o;
                    } else {
                        *reinterpret_cast<floatx4*>(static_cast<float*>(g.C) + off) = v;
                    }
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int nn = n + u;
                        if (nn >= g.N) break;
                        const int64_t off = (int64_t)(nn / g.seg_w) * g.seg_stride + (int64_t)m * g.ldc + nn % g.seg_w;
                        if (BF16OUT)
                            static_cast<__bf16*>(g.C)[off] = (__bf16)v[u];
                        else
                            static_cast<float*>(g.C)[off] = v[u];
                    }
                }
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, bool VEC, int GBK = 32, int NACC = 1>
hipError_t launch_cfg(const GemmArgs& g, hipStream_t s) {
    const int64_t tiles = (int64_t)((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    if (tiles <= 0 || tiles > 0x7fffffff) return hipErrorInvalidConfiguration;
    constexpr int NT = Cfg<BM, BN, WM, WN, GBK>::NT;
    const dim3 grid((unsigned)tiles), block(NT);
    const bool kf = VEC && g.K % GBK == 0;
    if (g.out_bf16) {
        if (kf)
            hipLaunchKernelGGL((gemm_bias_kernel<BM, BN, WM, WN, GBK, NACC, VEC, true, VEC>), grid, block, 0, s, g);
        else
            hipLaunchKernelGGL((gemm_bias_kernel<BM, BN, WM, WN, GBK, NACC, VEC, true, false>), grid, block, 0, s, g);
    } else {
        if (kf)
            hipLaunchKernelGGL((gemm_bias_kernel<BM, BN, WM, WN, GBK, NACC, VEC, false, VEC>), grid, block, 0, s, g);
        else
            hipLaunchKernelGGL((gemm_bias_kernel<BM, BN, WM, WN, GBK, NACC, VEC, false, false>), grid, block, 0, s, g);
    }
    return hipGetLastError();
}

// One tile shape for every problem: 64 x 128 outputs per workgroup, eight
// waves of 32 x 32, k-tiles of 32.  Measured on MI355X against 128x64,
// 64x64, 128x128, 32x64, 64x32 and 128x64/8-wave tiles, k-tiles of 16 and
// 64 and two accumulator chains: best or within noise on every projection
// shape of the c1 and c3 layers (more resident waves beat larger per-wave
// tiles).  With the VALU-free k loop, 128x128 (32x64 or 64x32 per wave),
// 64x128 (32x64 per wave) and 128x64 were again 1-68% slower, and so were
// the four-wave 64x64, 32x128 and 128x32 tiles (1-12%, also on the c1
// output projection's one-workgroup-per-CU grid).
template <bool VEC>
hipError_t launch_vec(const GemmArgs& g, hipStream_t s) {
    return launch_cfg<64, 128, 32, 32, VEC>(g, s);
}

}  // namespace

bool gemm_vec_ok(const GemmArgs& g) {
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    // 32-bit buffer offsets: W rows up to K + 64, A rows up to 128 past a tile's first row
    const int64_t wbytes = ((int64_t)(g.K + 64) * g.ldw + 128) * 4;
    const int64_t abytes = ((int64_t)128 * g.lda + g.K + 128) * 4;
    return al(g.A) && al(g.W) && al(g.C) && (!g.bias || al(g.bias)) && g.K % 4 == 0 && g.N % 4 == 0 &&
           g.lda % 4 == 0 && g.ldw % 4 == 0 && g.ldc % 4 == 0 && g.seg_w % 4 == 0 && g.seg_stride % 4 == 0 &&
           wbytes < ((int64_t)1 << 31) && abytes < ((int64_t)1 << 31);
}

hipError_t launch_gemm(const GemmArgs& g, hipStream_t s) {
    return gemm_vec_ok(g) ? launch_vec<true>(g, s) : launch_vec<false>(g, s);
}

}  // namespace hipgpt
