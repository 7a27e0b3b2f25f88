// rowtiles.h -- row-major LDS operand tiles for MFMA kernels that split the
// head dim over several waves (the wide attention backward, bwd_wide.h, and
// the wide forward, fa_wide.hip).
//
// A tile is 32 rows (queries or keys) of DP floats at pitch DP + 4.  The DH
// waves of a sub-block each own DW = DP / DH of the head dims.  Products that
// contract over the head dim (scores, dP) are formed per wave over its own
// dims and summed through LDS (publish / total); products that contract over
// the tile's 32 rows (P V, dS K, ...) read the row-major tile one row per
// MFMA step, 32 consecutive head dims across the lanes.
//
// MFMA 32x32x2 f32 operand layout (lane l, c = l & 31, h = l >> 5):
//   A[m][k]: lane holds A[c][h]          B[k][n]: lane holds B[h][c]
//   D[m][n]: register r holds D[8*(r/4) + 4*h + (r%4)][c]
#pragma once

#include "common.h"
#include "fa_common.h"

namespace hipgpt {

using fa::BK;

template <int DP, int DH>
struct RowTiles {
    static constexpr int RP = DP + 4;     // row pitch (floats)
    static constexpr int ROW = BK * RP;   // floats of a row-major tile
    static constexpr int CPR = DP / 4;    // 16-byte chunks per row
    static constexpr int CPT = BK * CPR;  // chunks per tile
    static constexpr int DW = DP / DH;    // head dims per wave
    static constexpr int NDBW = DW / 32;  // 32-dim blocks per wave
    static_assert(DW % 32 == 0, "a wave holds whole 32-dim blocks");

    // acc[m = row c of rt][n = c] += sum over the wave's dims d of rt[c][d] b[d],
    // lane (c, h) taking d = dh*DW + h*DW/2 + s (b holds the lane's DW/2 values).
    __device__ __forceinline__ static void dchain(floatx16& acc, const float* rt, const float* b, int c, int hf,
                                                  int dh) {
        const float* rr = rt + c * RP + dh * DW + hf * (DW / 2);
#pragma unroll
        for (int j = 0; j < DW / 8; ++j) {
            const floatx4 kv = *reinterpret_cast<const floatx4*>(rr + 4 * j);
#pragma unroll
            for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[u], b[4 * j + u], acc, 0, 0, 0);
        }
    }
    // acc[n][db][m = d][n = c] += sum_k rm[k][d] x[n][k][c] over the 32 tile
    // rows k, for the wave's dim blocks (d = dh*DW + db*32 + c); x in
    // accumulator register order (register 4g + u <-> row 8g + 4h + u).
    template <int N>
    __device__ __forceinline__ static void rchain(floatx16 (*acc)[NDBW], const float* rm, const floatx16* x, int c,
                                                  int hf, int dh) {
#pragma unroll
        for (int db = 0; db < NDBW; ++db) {
            const float* p = rm + 4 * hf * RP + dh * DW + db * 32 + c;
            float av[16];
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int u = 0; u < 4; ++u) av[4 * g + u] = p[(8 * g + u) * RP];
#pragma unroll
            for (int t = 0; t < 16; ++t)
#pragma unroll
                for (int n = 0; n < N; ++n)
                    acc[n][db] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[t], x[n][t], acc[n][db], 0, 0, 0);
        }
    }
    // Sum of the DH partial dP tiles of sub-block sb, in wave order (every
    // wave of the sub-block gets the same bits).  xch: [NW][4][64] floatx4.
    // The caller has stored its own partial and passed a barrier.
    __device__ __forceinline__ static floatx16 total(const floatx16& mine, const floatx4* xch, int sb, int dh,
                                                     int lane) {
        floatx16 t;
#pragma unroll
        for (int r = 0; r < 16; ++r) t[r] = fa::kSumInit;
#pragma unroll
        for (int j = 0; j < DH; ++j) {
            floatx16 p;
            if (j == dh) {
                p = mine;
            } else {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const floatx4 v = xch[((sb * DH + j) * 4 + g) * 64 + lane];
#pragma unroll
                    for (int u = 0; u < 4; ++u) p[4 * g + u] = v[u];
                }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) t[r] += p[r];
        }
        return t;
    }
    __device__ __forceinline__ static void publish(const floatx16& mine, floatx4* xch, int wave, int lane) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
            xch[(wave * 4 + g) * 64 + lane] = floatx4{mine[4 * g], mine[4 * g + 1], mine[4 * g + 2], mine[4 * g + 3]};
    }
    // This lane's DW/2 values of row `row` (dims dh*DW + h*DW/2 ..), zero past
    // D or past the last row.
    __device__ __forceinline__ static void load_lane_row(float* dst, const float* x, int row, int S, int D, int64_t ts,
                                                         int dh, int hf) {
        const int d0 = dh * DW + hf * (DW / 2);
        const float* p = x + (int64_t)row * ts + d0;
#pragma unroll
        for (int s = 0; s < DW / 2; s += 4) {
            const floatx4 t = (row < S && d0 + s < D) ? *reinterpret_cast<const floatx4*>(p + s)
                                                      : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[s + j] = t[j];
        }
    }
};

// Stage loads: NTILE (1 or 2) row-major tiles of 32 rows (tile 0 from loader
// l0, tile 1 from l1), 16-byte chunks spread over the workgroup's NT threads,
// chunks at or past D read as zero.  store() writes them at pitch DP + 4,
// tile 1 at tile_floats after tile 0.
template <int DP, int NT, int NTILE>
struct RowStage {
    static constexpr int CPR = DP / 4;
    static constexpr int CPT = BK * CPR;
    static constexpr int PER = (NTILE * CPT + NT - 1) / NT;
    static_assert(NTILE == 1 || NTILE == 2, "one or two tiles per stage");
    static_assert(CPT % 64 == 0, "a wave's chunks all come from one tile");
    floatx4 v[PER];

    __device__ __forceinline__ void load(const RowLoader& l0, const RowLoader& l1, int row0, int D, int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + i * NT;
            if ((NTILE * CPT) % NT != 0 && f >= NTILE * CPT) break;
            const int second = f >= CPT;
            const int g = second ? f - CPT : f;
            const int row = row0 + g / CPR, cc = g % CPR;
            floatx4 t = __builtin_amdgcn_readfirstlane(second) ? l1.load(row, cc) : l0.load(row, cc);
            if (cc * 4 >= D) t = floatx4{0.f, 0.f, 0.f, 0.f};
            v[i] = t;
        }
    }
    __device__ __forceinline__ void store(float* dst, int tile_floats, int tid) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + i * NT;
            if ((NTILE * CPT) % NT != 0 && f >= NTILE * CPT) break;
            const int second = f >= CPT;
            const int g = second ? f - CPT : f;
            *reinterpret_cast<floatx4*>(dst + second * tile_floats + (g / CPR) * (DP + 4) + (g % CPR) * 4) = v[i];
        }
    }
};

}  // namespace hipgpt
