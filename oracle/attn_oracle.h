/*
 * attn_oracle.h -- CPU restatement of HipGPT's multi-head self-attention
 * forward (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the checker for the HIP path and the scalar CPU baseline
 * timed beside it.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product (hipgpt_amd/) never links it.
 *
 * Reference (aarnetalman/HipGPT, paths relative to the repository root):
 *   src/hip_kernels.cpp:263-325  flash_attention_kernel<HEAD_DIM>  -> ORACLE_FLASH
 *   src/hip_kernels.cpp:329-402  multihead_attention_kernel_fallback -> ORACLE_FALLBACK
 *   src/hip_kernels.cpp:404-451  launch_multihead_attention dispatch
 *                                -> oracle_launch_multihead_attention
 *   src/hip_kernels.cpp:70-154   launch_matmul / launch_matmul_add_bias
 *                                -> oracle_matmul_add_bias
 *
 * Pinning (what fixes each function independently of its own formula):
 *   oracle_attention_f64 ........ textbook softmax(QK^T/sqrt(D))V in double;
 *                                 pinned by invariants with closed-form answers
 *                                 (constant V, zero K -> prefix mean, S=1,
 *                                 causal row 0, last row causal==non-causal,
 *                                 huge scale -> argmax row) and by brute force
 *                                 on tiny inputs computed with numpy.
 *   ORACLE_FLASH / ORACLE_FALLBACK pinned against oracle_attention_f64 (<=1e-6
 *                                 on unit-variance inputs), against the same
 *                                 invariants, and against golden vectors
 *                                 produced by the reference's own HIP kernels
 *                                 (oracle/_ref build run on an MI355X).
 *   oracle_fill_normal .......... SplitMix64 + Box-Muller; pinned by the
 *                                 published SplitMix64 test vector and by
 *                                 moment checks.
 *   oracle_matmul_add_bias ...... bit-exact against the reference's own
 *                                matmul kernels (oracle/_ref on an MI355X),
 *                                exact on integer-valued inputs (every partial
 *                                sum representable), and within the dot-product
 *                                error bound of a double-precision product.
 *   Causal mode has no reference counterpart (the reference is non-causal,
 *   src/hip_kernels.cpp:287,:353): it is the reference arithmetic restricted to
 *   keys j <= i + (Sk - Sq), probs written as 0 above the diagonal.  Its last
 *   query row is pinned by the non-causal reference (they coincide there).
 *   The device-math rounding of the reference (ocml expf, __expf on v_exp_f32,
 *   rsqrtf on v_rsq_f32) is not reproduced bit for bit; it differs from libm
 *   by a few ulp, far below the 1e-4 gate: parity of those ulps is unpinned.
 */
#ifndef HIPGPT_ATTN_ORACLE_H
#define HIPGPT_ATTN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_FLASH = 0, ORACLE_FALLBACK = 1 };

/* Strided attention problem.  Element (b, s, h, d) of Q lives at
 * q[b*q_bs + s*q_ts + h*q_hs + d]; likewise for K, V, O.  probs, when not
 * NULL, is dense [B][H][Sq][Sk].  Causal masks keys j > i + (Sk - Sq). */
typedef struct {
    const float *q, *k, *v;
    float *o, *probs;
    int B, H, Sq, Sk, D;
    int64_t q_bs, q_ts, q_hs;
    int64_t k_bs, k_ts, k_hs;
    int64_t v_bs, v_ts, v_hs;
    int64_t o_bs, o_ts, o_hs;
    int causal;
    int variant;  /* ORACLE_FLASH or ORACLE_FALLBACK */
} oracle_attn_problem;

/* SplitMix64 step (Steele, Lea, Flood 2014). */
uint64_t oracle_splitmix64(uint64_t *state);
/* n i.i.d. N(0,1) values: SplitMix64 -> Box-Muller in double -> fp32. */
void oracle_fill_normal(uint64_t seed, float *out, size_t n);
/* fp32 -> bf16 -> fp32 with round-to-nearest-even (NaN kept quiet). */
void oracle_round_bf16(const float *in, float *out, size_t n);

/* Scalar fp32 restatement of one of the two reference kernels over every
 * (b,h) pair, split across nthreads host threads (nthreads <= 0: 1).
 * Returns 0, or -1 on an invalid problem. */
int oracle_attention(const oracle_attn_problem *p, int nthreads);
/* Same, restricted to the listed (b,h) pairs (pairs[2*i], pairs[2*i+1]);
 * used to time a bounded sample. */
int oracle_attention_pairs(const oracle_attn_problem *p, const int *pairs,
                           int npairs, int nthreads);

/* Textbook attention in double precision (no clamps, exact softmax). */
int oracle_attention_f64(const oracle_attn_problem *p, int nthreads);

/* Mirror of launch_multihead_attention (src/hip_kernels.cpp:404-451) on the
 * planar d_qkv = [Q|K|V], each [B*S][E]: same validation, same dispatch
 * (flash restatement when D in {32,64} and S <= 512, fallback otherwise).
 * Returns -1 where the reference aborts (H <= 0 or E % H != 0). */
int oracle_launch_multihead_attention(const float *qkv, float *out,
                                      float *probs, int B, int S, int E, int H,
                                      int causal, int nthreads);

/* Restatements of the reference's unfused single-head helpers
 * (src/hip_kernels.cpp:454-532; declared include/hip_kernels.h:44-46).
 * Q, K, V, O are [B*S][D]; scores / probs are [B*S][S]; non-causal. */
/* scaled_dot_product_kernel :455-466: s = (sum_d q*k) * rsqrt(D) */
void oracle_scaled_dot_product(const float *Q, const float *K, float *scores,
                               int B, int S, int D, int nthreads);
/* softmax_kernel :478-502: max from -1e30, expf, sum, * 1/max(sum, 1e-20) */
void oracle_softmax_rows(const float *scores, float *out, int B, int S,
                         int nthreads);
/* attention_weighted_sum_kernel :513-525: o[d] = sum_j p_j * v_j[d] */
void oracle_attention_weighted_sum(const float *P, const float *V, float *out,
                                   int B, int S, int D, int nthreads);

/* Restatement of multihead_attention_backward_kernel + its launcher
 * (src/hip_kernels.cpp:1159-1272) on the planar buffers: grad_qkv is
 * [3][B*S][E] (dQ, dK, dV planes), fully overwritten (the launcher memsets
 * it, :1260).  Per (b, h, query i), in the kernel's order:
 *   pass 1 :1193-1200  ws = sum_j p_ij (gho . v_j)
 *   pass 2 :1208-1242  g = p_ij (gho . v_j - ws); dV_j += p_ij gho;
 *                      dQ_i += g k_j / sqrt(D); dK_j += g q_i / sqrt(D)
 * Sums into dK/dV are made in (i, j) order here; the kernel's atomics add
 * in an unspecified order (few-ulp differences, unpinned). */
int oracle_mha_backward(const float *grad_out, const float *qkv,
                        const float *probs, float *grad_qkv, int B, int S,
                        int E, int H);
/* The same on `nthreads` host threads, (b, h) pairs dealt round-robin:
 * distinct pairs write disjoint elements, so the result is identical. */
int oracle_mha_backward_mt(const float *grad_out, const float *qkv,
                           const float *probs, float *grad_qkv, int B, int S,
                           int E, int H, int nthreads);

/* Restatement of matmul_add_bias_tiled_kernel (src/hip_kernels.cpp:113-143;
 * bias == NULL: matmul_tiled_kernel, :70-100): A [M][N], B [N][K], C [M][K]
 * row-major; C = sequential fmaf sum over n, then + bias[col].  M <= 0 or
 * K <= 0 writes nothing (the reference's grid is empty).  Returns 0. */
int oracle_matmul_add_bias(const float *A, const float *B, const float *bias,
                           float *C, int M, int N, int K);

#ifdef __cplusplus
}
#endif
#endif
