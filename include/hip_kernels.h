#pragma once
// hip_kernels.h -- drop-in declarations of HipGPT's attention launchers and
// of the GEMMs either side of the attention.
//
// The signature is the one HipGPT declares in include/hip_kernels.h:39-43
// (C++ linkage; exported as _Z26launch_multihead_attentionPKfPfS1_iiii), so
// TransformerLayer::self_attention_forward (src/transformer_layer.cpp:218-219)
// links against libhipgpt_attn.so unchanged.  HipGPT's other declarations in
// that header (GEMM, layer norm, loss, optimisers, embeddings) are not
// provided by this library.

#include <hip/hip_runtime.h>

// Multi-head self-attention forward over HipGPT's planar packed buffer.
//   d_qkv        [3][B*S][E] fp32: Q, K, V planes at offsets 0, B*S*E, 2*B*S*E;
//                head h occupies columns [h*D, (h+1)*D), D = E / H.
//   d_output     [B*S][E] fp32, fully written.
//   d_attn_probs [B][H][S][S] fp32 normalised probabilities, written when
//                non-null (HipGPT always passes one; its backward reads it).
// Non-causal softmax(Q K^T / sqrt(D)) V per (batch, head).  Asynchronous on
// the null stream; allocates nothing.  Prints "Bad MHA config" and aborts
// when H <= 0 or E % H != 0, as the reference launcher does
// (src/hip_kernels.cpp:410-413).  Replaces src/hip_kernels.cpp:404-451.
void launch_multihead_attention(
    const float* d_qkv,
    float* d_output,
    float* d_attn_probs,
    int B, int S, int E, int H);

// HipGPT's unfused single-head helpers (include/hip_kernels.h:44-46,
// src/hip_kernels.cpp:454-532).  Q, K, V, output are [B*S][D]; scores and
// softmax are [B*S][S]; non-causal; fp32; asynchronous on the null stream;
// allocate nothing.  Non-positive sizes launch nothing.
//   scores = (Q K^T) * rsqrt(D)            per batch b
//   softmax_out = row softmax of scores    (max-subtracted, sum clamped >= 1e-20)
//   output = softmax V                     per batch b
void launch_scaled_dot_product(const float* Q, const float* K, float* scores, int B, int S, int D);
void launch_softmax(const float* scores, float* softmax_out, int B, int S);
void launch_attention_weighted_sum(const float* softmax, const float* V, float* output, int B, int S, int D);

// Attention backward on the forward's probabilities (include/hip_kernels.h:59-62,
// src/hip_kernels.cpp:1159-1272; called from TransformerLayer::backward,
// src/transformer_layer.cpp:285-286).
//   d_grad_attn_output dO [B*S][E]; d_qkv the forward's planar [Q|K|V];
//   d_softmax the forward's probs [B][H][S][S]; d_grad_qkv receives the planar
//   [dQ|dK|dV], every element written (the reference memsets, then adds).
// Non-causal as the reference; a causal forward's zero upper triangle gives the
// causal gradient.  Asynchronous on the null stream.  Uses a B*H*S float
// workspace cached per device (allocated on first use and when it must grow).
// Aborts with "Bad MHA config" when H <= 0 or E % H != 0.
void launch_multihead_attention_backward(
    const float* d_grad_attn_output, const float* d_qkv, const float* d_softmax,
    float* d_grad_qkv, int B, int S, int E, int H
);

// fp32 GEMMs of the projections either side of the attention
// (include/hip_kernels.h:6-7; src/hip_kernels.cpp:70-154; called from
// TransformerLayer::self_attention_forward, src/transformer_layer.cpp:217
// (QKV, N = E, K = 3E) and :220 (output projection, N = K = E)).
//   A [M][N], B [N][K], bias [K], C [M][K], all row-major fp32:
//   C = A B (+ bias), on fp32 MFMA.  Asynchronous on the null stream;
//   allocate nothing; M <= 0 or K <= 0 launches nothing; N <= 0 gives
//   C = bias (zero for launch_matmul), as the reference's loop does.
void launch_matmul(const float* A, const float* B, float* C, int M, int N, int K);
void launch_matmul_add_bias(const float* A, const float* B, const float* bias, float* C, int M, int N, int K);
