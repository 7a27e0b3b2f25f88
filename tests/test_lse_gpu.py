"""GPU parity tests of the probs-free training pair (hipgpt_attn_fwd_lse_qkv_planar
/ hipgpt_attn_bwd_lse_qkv_planar): the forward keeps a per-row log-sum-exp
instead of the [B][H][S][S] probs, the backward recomputes P from it.

HipGPT has no such pair (its backward reads the stored probs,
src/hip_kernels.cpp:1159-1272), so parity is anchored on what the pair must
reproduce:
  * lse against its closed form ln sum_j exp(q.k/sqrt(D)) in float64;
  * O against the oracle restatement of the reference forward;
  * the gradients against the oracle restatement of the reference backward
    (oracle_mha_backward) fed the oracle's probs -- the same function computed
    from the stored probs -- and against the GPU's own probs-based backward;
  * and against float64 torch autograd of the attention on the CPU.
Bars: lse 1e-5 (absolute, values O(5)); O 1e-4; gradients
1e-4 x max(1, max |gradient|), as for the probs-based backward.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hipgpt_amd import attention as A

pytestmark = pytest.mark.gpu


def dev_t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def tol(want):
    return 1e-4 * max(1.0, float(np.abs(want).max()))


def lse_f64(qkv, B, S, E, H, causal):
    """ln sum_j exp(q_i . k_j / sqrt(D)) per (b, h, i) in float64."""
    D = E // H
    x = qkv.astype(np.float64).reshape(3, B, S, H, D)
    q, k = x[0].transpose(0, 2, 1, 3), x[1].transpose(0, 2, 1, 3)
    s = q @ k.transpose(0, 1, 3, 2) / np.sqrt(D)
    if causal:
        s = np.where(np.triu(np.ones((S, S), dtype=bool), 1), -np.inf, s)
    m = s.max(-1, keepdims=True)
    return (m[..., 0] + np.log(np.exp(s - m).sum(-1))).reshape(B * H * S)


def run_pair(qkv, go, B, S, E, H, causal):
    d_qkv = dev_t(qkv)
    out = torch.full((B * S, E), float("nan"), device="cuda")
    lse = torch.full((B * H * S,), float("nan"), device="cuda")
    A.fwd_lse_qkv_planar(d_qkv, out, lse, B, S, E, H, causal=causal)
    grad = torch.full((3 * B * S * E,), float("nan"), device="cuda")
    A.bwd_lse_qkv_planar(dev_t(go), d_qkv, out, lse, grad, B, S, E, H, causal=causal)
    return d_qkv, out, lse, grad


# D = 32 and 64; S below, on and across the 32-row tile and the 128-query
# workgroup block; several heads and sequences.  S <= 256 runs the
# one-workgroup-per-(b, h) kernels (D = 32: S = 1, 7, 32, 45, 100, 255, 256;
# D = 64: S = 1, 33, 64, 130, 200, 256), S = 257 the query/key-stationary pair.
SHAPES = [(1, 1, 32, 1), (2, 7, 64, 2), (1, 33, 128, 2), (2, 64, 256, 4), (1, 100, 128, 4), (2, 130, 64, 1),
          (1, 256, 512, 8), (3, 45, 256, 8), (2, 32, 64, 2), (1, 255, 128, 4), (2, 256, 64, 2), (1, 257, 64, 2),
          (1, 1, 64, 1), (2, 200, 128, 2), (1, 257, 128, 2),
          (4, 64, 2560, 80)]  # B*H = 320 workgroups: more than one per CU


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,S,E,H", SHAPES)
def test_lse_pair_matches_oracle(dev, B, S, E, H, causal):
    qkv = O.seeded_planar(0x4C5345 + B * 131 + S * 7 + E, B, S, E)
    go = O.fill_normal(0x5EED + S + E, B * S * E)
    _, out, lse, grad = run_pair(qkv, go, B, S, E, H, causal)

    assert np.abs(host(lse) - lse_f64(qkv, B, S, E, H, causal)).max() <= 1e-5
    want_o, probs = O.launch_multihead_attention(qkv, B, S, E, H, causal=causal, want_probs=True)
    assert np.abs(host(out).reshape(-1) - want_o.reshape(-1)).max() <= 1e-4
    want_g = O.mha_backward(go, qkv, probs, B, S, E, H)
    got = host(grad)
    assert np.isfinite(got).all()  # every element written
    assert np.abs(got - want_g).max() <= tol(want_g)


# Head dims other than 32 / 64 (multiples of 4 up to 256): the forward's
# padded kernels (D = 16, 48, 80: padded to 32, 64, 128), D = 128 and the
# head-dim-split forward above 128; the backward's head-dim-split kernels,
# which pass the row dots dO . O through the B*H*S workspace.
WIDE_SHAPES = [(2, 40, 32, 2), (1, 70, 96, 2), (2, 33, 160, 2), (1, 130, 256, 2), (2, 100, 384, 3),
               (1, 257, 256, 1), (1, 64, 320, 2), (2, 150, 512, 2), (1, 1, 256, 2)]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,S,E,H", WIDE_SHAPES)
def test_lse_pair_other_head_dims(dev, B, S, E, H, causal):
    qkv = O.seeded_planar(0x57 + B * 131 + S * 7 + E, B, S, E)
    go = O.fill_normal(0x58 + S + E, B * S * E)
    _, out, lse, grad = run_pair(qkv, go, B, S, E, H, causal)
    assert np.abs(host(lse) - lse_f64(qkv, B, S, E, H, causal)).max() <= 1e-5
    want_o, probs = O.launch_multihead_attention(qkv, B, S, E, H, causal=causal, want_probs=True)
    assert np.abs(host(out).reshape(-1) - want_o.reshape(-1)).max() <= 1e-4
    want_g = O.mha_backward(go, qkv, probs, B, S, E, H)
    got = host(grad)
    assert np.isfinite(got).all()  # every element written
    assert np.abs(got - want_g).max() <= tol(want_g)


@pytest.mark.parametrize("causal", [True, False])
def test_lse_pair_matches_probs_backward_and_autograd(dev, causal):
    B, S, E, H = 2, 80, 256, 4
    D = E // H
    qkv = O.seeded_planar(77, B, S, E)
    go = O.fill_normal(78, B * S * E)
    d_qkv, out, _, grad = run_pair(qkv, go, B, S, E, H, causal)
    # the probs-based GPU backward on the same forward
    probs = torch.empty((B, H, S, S), device=dev)
    out2 = torch.empty((B * S, E), device=dev)
    A.qkv_planar(d_qkv, out2, probs, B, S, E, H, causal=causal)
    grad2 = torch.empty(3 * B * S * E, device=dev)
    A.attention_backward(dev_t(go), d_qkv, probs, grad2, B, S, E, H, causal=causal)
    g1, g2 = host(grad), host(grad2)
    assert np.abs(g1 - g2).max() <= tol(g2)
    assert np.abs(host(out) - host(out2)).max() <= 1e-5
    # float64 autograd on the CPU
    x = torch.from_numpy(qkv.astype(np.float64)).requires_grad_(True)
    q, k, v = (t.reshape(B, S, H, D).transpose(1, 2) for t in x.reshape(3, B * S, E))
    s = q @ k.transpose(-1, -2).contiguous() / np.sqrt(D)
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    o = (torch.softmax(s, -1) @ v).transpose(1, 2).reshape(B * S, E)
    o.backward(torch.from_numpy(go.astype(np.float64)).reshape(B * S, E))
    want = x.grad.numpy()
    assert np.abs(g1 - want).max() <= tol(want)


@pytest.mark.parametrize("cfg,shape", [("c1", (32, 256, 256, 8)), ("c2", (32, 256, 512, 8)),
                                       ("c3", (8, 1024, 768, 12)), ("c4", (4, 2048, 2048, 16))])
def test_lse_pair_baseline_configs(dev, cfg, shape):
    """Full c1 .. c4 shapes (causal): the probs-free gradients equal the
    probs-based backward's on the same forward (c4: D = 128, the head-dim-split
    backward)."""
    B, S, E, H = shape
    qkv = O.seeded_planar(91 + E, B, S, E)
    go = O.fill_normal(92 + E, B * S * E)
    d_qkv, out, lse, grad = run_pair(qkv, go, B, S, E, H, True)
    probs = torch.empty((B, H, S, S), device=dev)
    out2 = torch.empty((B * S, E), device=dev)
    A.qkv_planar(d_qkv, out2, probs, B, S, E, H, causal=True)
    grad2 = torch.empty(3 * B * S * E, device=dev)
    A.attention_backward(dev_t(go), d_qkv, probs, grad2, B, S, E, H, causal=True)
    g1, g2 = host(grad), host(grad2)
    assert np.isfinite(g1).all()
    assert np.abs(g1 - g2).max() <= tol(g2)
    # lse of a few rows against the closed form (whole-tensor f64 is cheap at this size)
    want_lse = lse_f64(qkv, B, S, E, H, True)
    assert np.abs(host(lse) - want_lse).max() <= 1e-5
