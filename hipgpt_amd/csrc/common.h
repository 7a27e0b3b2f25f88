// common.h -- shared device types and helpers for the gfx950 attention path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hipgpt {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef unsigned short ushort8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();
constexpr float kInf = __builtin_inff();
// Running-max start value.  Finite (unlike -inf) so that the first rescale
// exp2(m_old - m_new) is exp2(-huge) = 0 rather than exp2(-inf + inf) = NaN;
// the same value the reference starts from (src/hip_kernels.cpp:279, :350).
constexpr float kMaxInit = -1e30f;

enum Dtype : int { kF32 = 0, kBF16 = 1 };

// Word 3 of a raw (stride 0) buffer resource on CDNA3/CDNA4: 32-bit data
// format.  Loads past num_records bytes return zero.
constexpr int kBufferFlags = 0x00020000;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Strided attention problem as the kernels see it.  Element (b, s, h, d) of
// a tensor X lives at X[b*x_bs + s*x_ts + h*x_hs + d] (elements of the input
// dtype).  probs, when not null, is dense fp32 [B][H][Sq][Sk].
struct AttnArgs {
    const void* q;
    const void* k;
    const void* v;
    float* o;
    float* probs;
    int64_t q_bs, q_ts, q_hs;
    int64_t k_bs, k_ts, k_hs;
    int64_t v_bs, v_ts, v_hs;
    int64_t o_bs, o_ts, o_hs;
    int B, H, Sq, Sk, D;
    int causal_off;  // causal: query i sees keys j <= i + causal_off (Sk - Sq)
    float qscale;    // softmax scale * log2(e), folded into Q
    int n_qblk;      // query blocks per (b,h)
    float* lse;      // optional [B*H][Sq]: ln sum_j exp(scale * q_i . k_j) over visible keys
    // Start stagger (set by the launcher): workgroups [0, stagger_slots) --
    // the first set the device holds at once -- delay their first loads by
    // their launch rank; 0 = no stagger.
    int stagger_slots;
    // Late-block Q prefetch (set by the launcher for causal grids larger
    // than the device holds at once): a workgroup of launch rank r touches
    // the Q rows of rank r + pf_ranks; 0 = none.
    int pf_ranks;
    // Causal launch order (set by the launcher): launch rank short_rank - 1
    // runs the shortest query block, the others the rest longest first; 0 =
    // plain longest-first (the zero-initialised default).
    int short_rank;
};

// 16-byte chunks of `rows` consecutive rows (row stride ts floats) through a
// buffer resource whose range ends at the slice's last row: rows past it read
// as zero.
struct RowLoader {
    __amdgpu_buffer_rsrc_t rs;
    int row_bytes;
    __device__ __forceinline__ void init(const float* base, int64_t ts, int S, int D) {
        rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, (int)(((int64_t)(S - 1) * ts + D) * 4),
                                               kBufferFlags);
        row_bytes = (int)(ts * 4);
    }
    __device__ __forceinline__ floatx4 load(int row, int col4) const {
        return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, row * row_bytes + col4 * 16, 0, 0));
    }
};

// exp2 on the transcendental unit (v_exp_f32): exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Exchange with the lane 32 positions away (the other half of the wave).
__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32); }

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m);
    return x;
}

// Bounded waits.  Kernels whose waves wait on LDS flags set by other waves of
// the workgroup (instead of a barrier) poll a bounded number of times, so a
// schedule mistake cannot hang the GPU.  A wait that runs out lets the wave go
// on with data that may never have been published; each such expiry is counted
// here (one counter per translation unit and device, a vector atomic) and the
// host reads the count through wait_expired_take().
static __device__ unsigned int g_wait_expired;

__device__ __forceinline__ void note_wait_expired() {
    __hip_atomic_fetch_add(&g_wait_expired, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Host: this translation unit's expiry count on the current device.  One
// thread reads it into g_wait_taken with a device-side atomic (an exchange for
// zero when `clear` is set, so no expiry between the read and the clear is
// lost), then a blocking copy on the null stream brings it back.  The count is
// exact only when no kernel of the library is still running on another stream
// (the null stream does not wait for non-blocking streams).
static __device__ unsigned int g_wait_taken;

static __global__ void wait_expired_take_kernel(int clear) {
    g_wait_taken = clear ? __hip_atomic_exchange(&g_wait_expired, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                         : __hip_atomic_load(&g_wait_expired, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

static inline hipError_t wait_expired_take(unsigned int* count, bool clear) {
    hipLaunchKernelGGL(wait_expired_take_kernel, dim3(1), dim3(1), 0, 0, clear ? 1 : 0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return hipMemcpyFromSymbol(count, HIP_SYMBOL(g_wait_taken), sizeof(unsigned int), 0, hipMemcpyDeviceToHost);
}

// Workgroups of kernel `kern` (block threads, dynamic LDS bytes) the current
// device holds at once: occupancy per CU times the CU count; 0 if unknown.
// The caller caches the value per device and kernel (static state of its own
// template instantiation).
inline int device_resident_slots(const void* kern, int block, size_t lds) {
    int dev = 0, per_cu = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, block, lds) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return per_cu > 0 && cus > 0 ? per_cu * cus : 0;
}

// Compute units of the current device (cached per device; 0 if unknown).
inline int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int v = __atomic_load_n(&cus[dev], __ATOMIC_RELAXED);
    if (v == 0 && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
        __atomic_store_n(&cus[dev], v, __ATOMIC_RELAXED);
    return v;
}

// Per-device cache of device_resident_slots for one kernel (a static of the
// launching template, so each kernel instantiation has its own).
struct ResidentSlots {
    int slots[64] = {};
    int get(const void* kern, int block, size_t lds) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
        int v = __atomic_load_n(&slots[dev], __ATOMIC_RELAXED);
        if (v == 0) {
            v = device_resident_slots(kern, block, lds);
            __atomic_store_n(&slots[dev], v, __ATOMIC_RELAXED);
        }
        return v;
    }
};

// Workgroups are dispatched to the 8 XCDs round-robin (id % 8), and each XCD
// has its own L2.  xcd_remap renumbers a 1-D grid so that XCD x runs the
// contiguous logical range [x*per, (x+1)*per), per = total / 8 (ids past
// 8*per keep their number): neighbouring logical workgroups, which share
// operands, then share one L2.  A bijection on [0, total).
__device__ __forceinline__ int xcd_remap(int id, int total) {
    const int per = total / 8;
    if (id >= 8 * per) return id;
    return (id % 8) * per + id / 8;
}

}  // namespace hipgpt
