/*
 * attn_oracle.c -- scalar CPU restatement of HipGPT's attention forward.
 *
 * TEST INFRASTRUCTURE: the checker for the HIP path and the CPU baseline
 * timed beside it; never part of the product.  The header lists what pins
 * each function.
 *
 * Built with -O2 -mfma and without -ffast-math: fmaf() becomes one fused
 * multiply-add, matching the contraction clang applies to the reference's
 * `acc += a * b` loops on the GPU, and all sums run in the reference's
 * sequential order.
 */
#include "attn_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ RNG */

uint64_t oracle_splitmix64(uint64_t *state)
{
    uint64_t z = (*state += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* Uniform double in (0, 1]: 53 random bits, shifted off zero. */
static double unit_open0(uint64_t *st)
{
    return ((double)(oracle_splitmix64(st) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

void oracle_fill_normal(uint64_t seed, float *out, size_t n)
{
    uint64_t st = seed;
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = 0;
    while (i < n) {
        double u1 = unit_open0(&st);
        double u2 = unit_open0(&st);
        double r = sqrt(-2.0 * log(u1));
        out[i++] = (float)(r * cos(two_pi * u2));
        if (i < n) out[i++] = (float)(r * sin(two_pi * u2));
    }
}

void oracle_round_bf16(const float *in, float *out, size_t n)
{
    for (size_t i = 0; i < n; ++i) {
        uint32_t u;
        memcpy(&u, &in[i], 4);
        if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) {
            u |= 0x00400000u; /* quiet NaN, keep payload top bits */
        } else {
            u += 0x7FFFu + ((u >> 16) & 1u); /* round to nearest even */
        }
        u &= 0xFFFF0000u;
        memcpy(&out[i], &u, 4);
    }
}

/* ------------------------------------------------------------- helpers */

static int problem_ok(const oracle_attn_problem *p)
{
    if (!p || !p->q || !p->k || !p->v || !p->o) return 0;
    if (p->B <= 0 || p->H <= 0 || p->Sq <= 0 || p->Sk <= 0 || p->D <= 0) return 0;
    if (p->causal && p->Sk < p->Sq) return 0;
    if (p->variant != ORACLE_FLASH && p->variant != ORACLE_FALLBACK) return 0;
    return 1;
}

/* Number of visible keys for query i: all Sk, or i + 1 + (Sk - Sq) causal. */
static int visible_keys(const oracle_attn_problem *p, int i)
{
    if (!p->causal) return p->Sk;
    int n = i + 1 + (p->Sk - p->Sq);
    return n < p->Sk ? n : p->Sk;
}

/* Head-dim scale.  The reference uses rsqrtf((float)D) (v_rsq_f32 on the
 * GPU, within 1 ulp of the correctly rounded value computed here). */
static float head_scale(int D) { return 1.0f / sqrtf((float)D); }

/* Sequential fused dot product: `dot += q[d] * k[d]` as contracted by clang
 * (src/hip_kernels.cpp:290-292, :355-356). */
static float dot_fma(const float *a, const float *b, int D)
{
    float acc = 0.0f;
    for (int d = 0; d < D; ++d) acc = fmaf(a[d], b[d], acc);
    return acc;
}

/* ------------------------------------------------ flash restatement (one
 * query row).  Follows flash_attention_kernel, src/hip_kernels.cpp:263-325:
 *   pass 1 :286-296  raw scores s_j = dot * scale, running fmaxf from -1e30
 *   pass 2 :298-304  e_j = expf(s_j - max), sequential sum, clamp >= 1e-20
 *   pass 3 :306-310  probs p_j = e_j / sum (IEEE divide) stored
 *   pass 4 :312-319  O[d] += p_j * v_j[d], p_j read back from probs
 * The kernel keeps scores in a per-thread array; here `scratch` has Sk
 * entries.  Causal restricts j to the visible prefix; masked probs are 0. */
static void flash_row(const oracle_attn_problem *p, int b, int h, int i,
                      float *scratch, float *acc)
{
    const int D = p->D, Sk = p->Sk, nvis = visible_keys(p, i);
    const float scale = head_scale(D);
    const float *q = p->q + b * p->q_bs + (int64_t)i * p->q_ts + h * p->q_hs;
    float *o = p->o + b * p->o_bs + (int64_t)i * p->o_ts + h * p->o_hs;
    float *prow = p->probs
        ? p->probs + (((int64_t)b * p->H + h) * p->Sq + i) * (int64_t)Sk
        : NULL;

    float mx = -1e30f;
    for (int j = 0; j < nvis; ++j) {
        const float *k = p->k + b * p->k_bs + (int64_t)j * p->k_ts + h * p->k_hs;
        float s = dot_fma(q, k, D) * scale;
        scratch[j] = s;
        mx = fmaxf(mx, s);
    }
    float sum = 0.0f;
    for (int j = 0; j < nvis; ++j) {
        float e = expf(scratch[j] - mx);
        scratch[j] = e;
        sum += e;
    }
    sum = fmaxf(sum, 1e-20f);
    for (int j = 0; j < nvis; ++j) scratch[j] = scratch[j] / sum;
    if (prow) {
        memcpy(prow, scratch, (size_t)nvis * sizeof(float));
        for (int j = nvis; j < Sk; ++j) prow[j] = 0.0f;
    }
    for (int d = 0; d < D; ++d) acc[d] = 0.0f;
    for (int j = 0; j < nvis; ++j) {
        const float *v = p->v + b * p->v_bs + (int64_t)j * p->v_ts + h * p->v_hs;
        const float pj = scratch[j];
        for (int d = 0; d < D; ++d) acc[d] = fmaf(pj, v[d], acc[d]);
    }
    for (int d = 0; d < D; ++d) o[d] = acc[d];
}

/* --------------------------------------------- fallback restatement (one
 * query row).  Follows multihead_attention_kernel_fallback,
 * src/hip_kernels.cpp:329-402:
 *   pass 1 :349-360  max of dot * inv_sqrt, strict `>` update from -1e30
 *   pass 2 :362-374  recompute dot, sum of __expf(s - max), clamp >= 1e-20,
 *                    inv_sum = 1 / sum
 *   pass 3 :376-401  recompute dot, p = __expf(s - max) * inv_sum, optional
 *                    probs store, O[d] += p * v_j[d] accumulated in O itself
 * __expf is exp2(log2e * x) on the GPU; libm expf is used here (few-ulp
 * difference, unpinned). */
static void fallback_row(const oracle_attn_problem *p, int b, int h, int i)
{
    const int D = p->D, Sk = p->Sk, nvis = visible_keys(p, i);
    const float inv_sqrt = head_scale(D);
    const float *q = p->q + b * p->q_bs + (int64_t)i * p->q_ts + h * p->q_hs;
    float *o = p->o + b * p->o_bs + (int64_t)i * p->o_ts + h * p->o_hs;
    float *prow = p->probs
        ? p->probs + (((int64_t)b * p->H + h) * p->Sq + i) * (int64_t)Sk
        : NULL;

    float mx = -1e30f;
    for (int j = 0; j < nvis; ++j) {
        const float *k = p->k + b * p->k_bs + (int64_t)j * p->k_ts + h * p->k_hs;
        float s = dot_fma(q, k, D) * inv_sqrt;
        if (s > mx) mx = s;
    }
    float sum = 0.0f;
    for (int j = 0; j < nvis; ++j) {
        const float *k = p->k + b * p->k_bs + (int64_t)j * p->k_ts + h * p->k_hs;
        sum += expf(dot_fma(q, k, D) * inv_sqrt - mx);
    }
    sum = fmaxf(sum, 1e-20f);
    const float inv_sum = 1.0f / sum;
    for (int d = 0; d < D; ++d) o[d] = 0.0f;
    for (int j = 0; j < nvis; ++j) {
        const float *k = p->k + b * p->k_bs + (int64_t)j * p->k_ts + h * p->k_hs;
        const float *v = p->v + b * p->v_bs + (int64_t)j * p->v_ts + h * p->v_hs;
        float pj = expf(dot_fma(q, k, D) * inv_sqrt - mx) * inv_sum;
        if (prow) prow[j] = pj;
        for (int d = 0; d < D; ++d) o[d] = fmaf(pj, v[d], o[d]);
    }
    if (prow)
        for (int j = nvis; j < Sk; ++j) prow[j] = 0.0f;
}

/* ------------------------------------------ fp64 textbook closed form */
static void f64_row(const oracle_attn_problem *p, int b, int h, int i,
                    double *scratch, double *acc)
{
    const int D = p->D, Sk = p->Sk, nvis = visible_keys(p, i);
    const double scale = 1.0 / sqrt((double)D);
    const float *q = p->q + b * p->q_bs + (int64_t)i * p->q_ts + h * p->q_hs;
    float *o = p->o + b * p->o_bs + (int64_t)i * p->o_ts + h * p->o_hs;
    double mx = -INFINITY;
    for (int j = 0; j < nvis; ++j) {
        const float *k = p->k + b * p->k_bs + (int64_t)j * p->k_ts + h * p->k_hs;
        double s = 0.0;
        for (int d = 0; d < D; ++d) s += (double)q[d] * (double)k[d];
        s *= scale;
        scratch[j] = s;
        if (s > mx) mx = s;
    }
    double sum = 0.0;
    for (int j = 0; j < nvis; ++j) {
        scratch[j] = exp(scratch[j] - mx);
        sum += scratch[j];
    }
    for (int d = 0; d < D; ++d) acc[d] = 0.0;
    for (int j = 0; j < nvis; ++j) {
        const float *v = p->v + b * p->v_bs + (int64_t)j * p->v_ts + h * p->v_hs;
        double pj = scratch[j] / sum;
        for (int d = 0; d < D; ++d) acc[d] += pj * (double)v[d];
    }
    for (int d = 0; d < D; ++d) o[d] = (float)acc[d];
    if (p->probs) {
        float *prow = p->probs + (((int64_t)b * p->H + h) * p->Sq + i) * (int64_t)Sk;
        for (int j = 0; j < nvis; ++j) prow[j] = (float)(scratch[j] / sum);
        for (int j = nvis; j < Sk; ++j) prow[j] = 0.0f;
    }
}

/* ------------------------------------------------------- thread pool */

typedef struct {
    const oracle_attn_problem *p;
    const int *pairs; /* NULL: all (b,h) */
    int npairs;
    int tid, nthreads;
    int f64;
    int status;
} worker_arg;

static void *worker(void *argp)
{
    worker_arg *a = (worker_arg *)argp;
    const oracle_attn_problem *p = a->p;
    const size_t nscr = (size_t)p->Sk > (size_t)p->D ? (size_t)p->Sk : (size_t)p->D;
    void *scr = malloc(nscr * sizeof(double));
    void *acc = malloc((size_t)p->D * sizeof(double));
    if (!scr || !acc) {
        free(scr);
        free(acc);
        a->status = -1;
        return NULL;
    }
    for (int idx = a->tid; idx < a->npairs; idx += a->nthreads) {
        int b, h;
        if (a->pairs) {
            b = a->pairs[2 * idx];
            h = a->pairs[2 * idx + 1];
        } else {
            b = idx / p->H;
            h = idx % p->H;
        }
        for (int i = 0; i < p->Sq; ++i) {
            if (a->f64)
                f64_row(p, b, h, i, (double *)scr, (double *)acc);
            else if (p->variant == ORACLE_FLASH)
                flash_row(p, b, h, i, (float *)scr, (float *)acc);
            else
                fallback_row(p, b, h, i);
        }
    }
    free(scr);
    free(acc);
    a->status = 0;
    return NULL;
}

static int run_pool(const oracle_attn_problem *p, const int *pairs, int npairs,
                    int nthreads, int f64)
{
    if (!problem_ok(p)) return -1;
    if (pairs) {
        for (int i = 0; i < npairs; ++i)
            if (pairs[2 * i] < 0 || pairs[2 * i] >= p->B || pairs[2 * i + 1] < 0 ||
                pairs[2 * i + 1] >= p->H)
                return -1;
    }
    if (nthreads <= 0) nthreads = 1;
    if (nthreads > npairs) nthreads = npairs > 0 ? npairs : 1;
    worker_arg *args = (worker_arg *)calloc((size_t)nthreads, sizeof(worker_arg));
    pthread_t *th = (pthread_t *)calloc((size_t)nthreads, sizeof(pthread_t));
    if (!args || !th) {
        free(args);
        free(th);
        return -1;
    }
    for (int t = 0; t < nthreads; ++t) {
        args[t] = (worker_arg){p, pairs, npairs, t, nthreads, f64, -1};
    }
    int rc = 0;
    if (nthreads == 1) {
        worker(&args[0]);
    } else {
        for (int t = 0; t < nthreads; ++t)
            if (pthread_create(&th[t], NULL, worker, &args[t]) != 0) {
                args[t].status = -1;
                th[t] = 0;
            }
        for (int t = 0; t < nthreads; ++t)
            if (th[t]) pthread_join(th[t], NULL);
    }
    for (int t = 0; t < nthreads; ++t)
        if (args[t].status != 0) rc = -1;
    free(args);
    free(th);
    return rc;
}

int oracle_attention(const oracle_attn_problem *p, int nthreads)
{
    if (!problem_ok(p)) return -1;
    return run_pool(p, NULL, p->B * p->H, nthreads, 0);
}

int oracle_attention_pairs(const oracle_attn_problem *p, const int *pairs,
                           int npairs, int nthreads)
{
    if (!pairs || npairs < 0) return -1;
    return run_pool(p, pairs, npairs, nthreads, 0);
}

int oracle_attention_f64(const oracle_attn_problem *p, int nthreads)
{
    if (!problem_ok(p)) return -1;
    return run_pool(p, NULL, p->B * p->H, nthreads, 1);
}

/* Planar d_qkv split and dispatch, src/hip_kernels.cpp:404-451. */
int oracle_launch_multihead_attention(const float *qkv, float *out,
                                      float *probs, int B, int S, int E, int H,
                                      int causal, int nthreads)
{
    if (H <= 0 || (E % H) != 0) return -1; /* :410-413 aborts here */
    const int64_t plane = (int64_t)B * S * E;  /* :415-417 */
    const int D = E / H;
    oracle_attn_problem p;
    memset(&p, 0, sizeof(p));
    p.q = qkv;
    p.k = qkv + plane;
    p.v = qkv + 2 * plane;
    p.o = out;
    p.probs = probs;
    p.B = B;
    p.H = H;
    p.Sq = S;
    p.Sk = S;
    p.D = D;
    p.q_bs = p.k_bs = p.v_bs = p.o_bs = (int64_t)S * E;
    p.q_ts = p.k_ts = p.v_ts = p.o_ts = E;
    p.q_hs = p.k_hs = p.v_hs = p.o_hs = D;
    p.causal = causal;
    p.variant = ((D == 64 || D == 32) && S <= 512) ? ORACLE_FLASH : ORACLE_FALLBACK; /* :422 */
    return oracle_attention(&p, nthreads);
}

/* ------------------------------------------------- unfused helpers
 * Restated from src/hip_kernels.cpp:454-532 (one thread per token there,
 * one row per loop iteration here; same per-element arithmetic). */

typedef struct {
    const float *a, *b;
    float *out;
    int B, S, D, kind, tid, nthreads;
} helper_arg;

static void *helper_worker(void *argp)
{
    const helper_arg *h = (const helper_arg *)argp;
    const int S = h->S, D = h->D;
    const int64_t rows = (int64_t)h->B * S;
    for (int64_t t = h->tid; t < rows; t += h->nthreads) {
        const int64_t base = (t / S) * (int64_t)S * D; /* (token / S) * S * D */
        if (h->kind == 0) {                             /* scaled dot product */
            const float inv = 1.0f / sqrtf((float)D);
            for (int j = 0; j < S; ++j) {
                float sum = 0.0f;
                for (int d = 0; d < D; ++d)
                    sum = fmaf(h->a[t * D + d], h->b[base + (int64_t)j * D + d], sum);
                h->out[t * S + j] = sum * inv;
            }
        } else if (h->kind == 1) {                      /* softmax row */
            const float *row = h->a + t * S;
            float *o = h->out + t * S;
            float mx = -1e30f;
            for (int j = 0; j < S; ++j) mx = fmaxf(mx, row[j]);
            float sum = 0.0f;
            for (int j = 0; j < S; ++j) {
                o[j] = expf(row[j] - mx);
                sum += o[j];
            }
            const float inv = 1.0f / fmaxf(sum, 1e-20f);
            for (int j = 0; j < S; ++j) o[j] *= inv;
        } else {                                        /* weighted sum */
            for (int d = 0; d < D; ++d) {
                float sum = 0.0f;
                for (int j = 0; j < S; ++j)
                    sum = fmaf(h->a[t * S + j], h->b[base + (int64_t)j * D + d], sum);
                h->out[t * D + d] = sum;
            }
        }
    }
    return NULL;
}

static void helper_run(const float *a, const float *b, float *out, int B, int S,
                       int D, int kind, int nthreads)
{
    if (B <= 0 || S <= 0 || (kind != 1 && D <= 0)) return;
    if (nthreads <= 0) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    pthread_t th[64];
    helper_arg args[64];
    for (int t = 0; t < nthreads; ++t)
        args[t] = (helper_arg){a, b, out, B, S, D, kind, t, nthreads};
    int started[64] = {0};
    for (int t = 1; t < nthreads; ++t)
        started[t] = pthread_create(&th[t], NULL, helper_worker, &args[t]) == 0;
    helper_worker(&args[0]);
    for (int t = 1; t < nthreads; ++t) {
        if (started[t])
            pthread_join(th[t], NULL);
        else
            helper_worker(&args[t]);
    }
}

void oracle_scaled_dot_product(const float *Q, const float *K, float *scores,
                               int B, int S, int D, int nthreads)
{
    helper_run(Q, K, scores, B, S, D, 0, nthreads);
}

void oracle_softmax_rows(const float *scores, float *out, int B, int S,
                         int nthreads)
{
    helper_run(scores, NULL, out, B, S, 0, 1, nthreads);
}

void oracle_attention_weighted_sum(const float *P, const float *V, float *out,
                                   int B, int S, int D, int nthreads)
{
    helper_run(P, V, out, B, S, D, 2, nthreads);
}

/* ---------------------------------------------------- attention backward */
typedef struct {
    const float *grad_out, *qkv, *probs;
    float *grad_qkv;
    int B, S, E, H, tid, nthreads;
} bwd_arg;

/* One (b, h): the kernel's threads (b, i, h) for i = 0..S-1, in order.
 * Every write lands in head h's columns of batch b's rows, so distinct
 * (b, h) pairs never touch the same element. */
static void mha_backward_pair(const bwd_arg *a, int b, int h)
{
    const int S = a->S, E = a->E, D = E / a->H;
    const int64_t plane = (int64_t)a->B * S * E;
    const float *Q = a->qkv, *K = a->qkv + plane, *V = a->qkv + 2 * plane;
    float *dQ = a->grad_qkv, *dK = a->grad_qkv + plane, *dV = a->grad_qkv + 2 * plane;
    const float inv = 1.0f / sqrtf((float)D);
    for (int i = 0; i < S; ++i) {
        const int64_t ti = (int64_t)b * S + i;
        const float *gho = a->grad_out + ti * E + h * D;
        const float *q = Q + ti * E + h * D;
        float *dq = dQ + ti * E + h * D;
        const float *prow = a->probs + (((int64_t)b * a->H + h) * S + i) * S;
        float ws = 0.0f;
        for (int j = 0; j < S; ++j) {
            const float *v = V + ((int64_t)b * S + j) * E + h * D;
            ws = fmaf(prow[j], dot_fma(gho, v, D), ws);
        }
        for (int j = 0; j < S; ++j) {
            const int64_t tj = (int64_t)b * S + j;
            const float *k = K + tj * E + h * D;
            const float *v = V + tj * E + h * D;
            const float pij = prow[j];
            const float g = pij * (dot_fma(gho, v, D) - ws);
            float *dv = dV + tj * E + h * D;
            float *dk = dK + tj * E + h * D;
            for (int d = 0; d < D; ++d) {
                dv[d] += pij * gho[d];
                dq[d] = fmaf(g * k[d], inv, dq[d]);
                dk[d] += g * q[d] * inv;
            }
        }
    }
}

static void *bwd_worker(void *argp)
{
    const bwd_arg *a = (const bwd_arg *)argp;
    for (int idx = a->tid; idx < a->B * a->H; idx += a->nthreads) mha_backward_pair(a, idx / a->H, idx % a->H);
    return NULL;
}

int oracle_mha_backward_mt(const float *grad_out, const float *qkv,
                           const float *probs, float *grad_qkv, int B, int S,
                           int E, int H, int nthreads)
{
    if (B <= 0 || S <= 0 || H <= 0 || E % H != 0) return -1;
    memset(grad_qkv, 0, (size_t)(3 * (int64_t)B * S * E) * sizeof(float));
    const int npairs = B * H;
    if (nthreads <= 0) nthreads = 1;
    if (nthreads > npairs) nthreads = npairs;
    bwd_arg *args = (bwd_arg *)calloc((size_t)nthreads, sizeof(bwd_arg));
    pthread_t *th = (pthread_t *)calloc((size_t)nthreads, sizeof(pthread_t));
    if (!args || !th) {
        free(args);
        free(th);
        return -2;
    }
    for (int t = 0; t < nthreads; ++t) args[t] = (bwd_arg){grad_out, qkv, probs, grad_qkv, B, S, E, H, t, nthreads};
    int started = 1;
    for (int t = 1; t < nthreads; ++t) {
        if (pthread_create(&th[t], NULL, bwd_worker, &args[t]) != 0) break;
        ++started;
    }
    bwd_worker(&args[0]);
    for (int t = 1; t < started; ++t) pthread_join(th[t], NULL);
    /* pairs of threads that could not start, on this thread */
    for (int t = started; t < nthreads; ++t) bwd_worker(&args[t]);
    free(args);
    free(th);
    return 0;
}

int oracle_mha_backward(const float *grad_out, const float *qkv,
                        const float *probs, float *grad_qkv, int B, int S,
                        int E, int H)
{
    return oracle_mha_backward_mt(grad_out, qkv, probs, grad_qkv, B, S, E, H, 1);
}

/* ------------------------------------------------------------------ GEMM */

/* matmul_tiled_kernel / matmul_add_bias_tiled_kernel (src/hip_kernels.cpp:
 * 70-100, :113-143): each output element is one thread's fp32 accumulator,
 * summed over n = 0..N-1 in order (the 32-wide LDS tiles only stage the
 * operands; the per-thread order is sequential) with the contracted
 * `sum += As*Bs` (one fused multiply-add), then `sum + bias[col]`. */
int oracle_matmul_add_bias(const float *A, const float *B, const float *bias,
                           float *C, int M, int N, int K)
{
    if (M <= 0 || K <= 0) return 0;
    for (int64_t row = 0; row < M; ++row) {
        for (int64_t col = 0; col < K; ++col) {
            float sum = 0.0f;
            for (int64_t n = 0; n < N; ++n) sum = fmaf(A[row * N + n], B[n * K + col], sum);
            C[row * K + col] = bias ? sum + bias[col] : sum;
        }
    }
    return 0;
}
