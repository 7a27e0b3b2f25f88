"""GPU parity tests: the HIP path (through the C ABI) against the oracle.

Bars: fp32 max-abs(O) <= 1e-4 on unit-variance inputs;
probabilities max-abs <= 1e-5.  The non-causal legacy launcher is also
compared with the reference's own HIP kernels (oracle/_ref) on the same
device buffers.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hipgpt_amd import attention as A

pytestmark = pytest.mark.gpu

TOL_O = 1e-4
TOL_P = 1e-5


def dev_t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


# (B, S, E, H): D = 32/64/128 MFMA fast path, padded D (16, 48, 96), generic
# D (7, 256), S below / across / not a multiple of the 32-row tile, S > 512.
LEGACY_SHAPES = [
    (1, 1, 32, 1), (2, 7, 64, 2), (1, 33, 128, 2), (2, 64, 256, 2), (1, 100, 96, 2),
    (1, 45, 32, 2), (1, 70, 192, 2), (1, 40, 512, 2), (1, 9, 14, 2), (2, 300, 256, 4),
    (1, 520, 64, 2), (1, 129, 128, 1),
]


@pytest.mark.parametrize("with_probs", [True, False])
@pytest.mark.parametrize("B,S,E,H", LEGACY_SHAPES)
def test_legacy_launcher_matches_oracle(dev, B, S, E, H, with_probs):
    qkv = O.seeded_planar(B * 7919 + S * 31 + E, B, S, E)
    want_o, want_p = O.launch_multihead_attention(qkv, B, S, E, H, want_probs=True)
    d_qkv = dev_t(qkv)
    d_out = torch.full((B * S, E), float("nan"), device=dev)
    d_p = torch.full((B, H, S, S), float("nan"), device=dev) if with_probs else None
    A.launch_multihead_attention(d_qkv, d_out, d_p, B, S, E, H)
    got = host(d_out)
    assert np.isfinite(got).all()
    assert np.abs(got - want_o).max() <= TOL_O
    if with_probs:
        assert np.abs(host(d_p) - want_p).max() <= TOL_P


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("with_probs", [True, False])
@pytest.mark.parametrize("B,S,E,H", [(2, 37, 64, 2), (1, 160, 128, 2), (2, 96, 256, 2), (1, 75, 96, 1),
                                     (1, 50, 512, 2)])
def test_planar_causal_matches_oracle(dev, B, S, E, H, causal, with_probs):
    qkv = O.seeded_planar(S * 13 + E, B, S, E)
    want_o, want_p = O.launch_multihead_attention(qkv, B, S, E, H, causal=causal, want_probs=True)
    d_out = torch.empty((B * S, E), device=dev)
    d_p = torch.full((B, H, S, S), float("nan"), device=dev) if with_probs else None
    A.qkv_planar(dev_t(qkv), d_out, d_p, B, S, E, H, causal=causal)
    assert np.abs(host(d_out) - want_o).max() <= TOL_O
    if with_probs:
        p = host(d_p)
        assert np.abs(p - want_p).max() <= TOL_P
        if causal:
            iu = np.triu_indices(S, 1)
            assert np.all(p[:, :, iu[0], iu[1]] == 0.0)


# 128..256 keys and few query tiles (D <= 32: at most 128, D = 64: at most
# 512): the launcher splits each query sub-block's keys over 4 waves
# (HipGPT's generation call, B = 1, H = 8, S = 256, at D = 32 and 64, is one
# such shape).  Padded D (16, 24, 48), ragged S, both masks, probs on and off;
# at D = 32 with probs a wave's keys span one stage (S = 128) or two (S = 129 ..
# 256), which are loaded together.
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("with_probs", [True, False])
@pytest.mark.parametrize("B,S,E,H", [(1, 256, 256, 8), (2, 129, 64, 2), (1, 200, 96, 4), (2, 128, 32, 2),
                                     (1, 250, 48, 2), (1, 256, 512, 8), (2, 150, 128, 2), (3, 130, 192, 4),
                                     (8, 256, 512, 8), (1, 128, 256, 8), (3, 160, 96, 3), (2, 255, 64, 2)])
def test_small_grid_key_split_matches_oracle(dev, B, S, E, H, causal, with_probs):
    qkv = O.seeded_planar(S * 17 + E + B, B, S, E)
    want_o, want_p = O.launch_multihead_attention(qkv, B, S, E, H, causal=causal, want_probs=True)
    d_out = torch.full((B * S, E), float("nan"), device=dev)
    d_p = torch.full((B, H, S, S), float("nan"), device=dev) if with_probs else None
    A.qkv_planar(dev_t(qkv), d_out, d_p, B, S, E, H, causal=causal)
    assert np.abs(host(d_out) - want_o).max() <= TOL_O
    if with_probs:
        assert np.abs(host(d_p) - want_p).max() <= TOL_P


# D = 64 with probs, 193 <= S <= 256 and B*H at least the CU count (256 on
# MI355X): the one-workgroup-per-(b, h) resident kernel, at ragged S; the
# same shapes without probs run the streaming kernel.
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("with_probs", [True, False])
@pytest.mark.parametrize("B,S,E,H", [(32, 200, 512, 8), (64, 250, 256, 4)])
def test_resident_kernel_matches_oracle(dev, B, S, E, H, causal, with_probs):
    qkv = O.seeded_planar(S * 19 + E + B, B, S, E)
    want_o, want_p = O.launch_multihead_attention(qkv, B, S, E, H, causal=causal, want_probs=True)
    d_out = torch.full((B * S, E), float("nan"), device=dev)
    d_p = torch.full((B, H, S, S), float("nan"), device=dev) if with_probs else None
    A.qkv_planar(dev_t(qkv), d_out, d_p, B, S, E, H, causal=causal)
    assert np.abs(host(d_out) - want_o).max() <= TOL_O
    if with_probs:
        assert np.abs(host(d_p) - want_p).max() <= TOL_P


def _ref_or_skip():
    if not O.ref_available():
        pytest.skip("reference build oracle/_ref missing")
    return O.ref_lib()


@pytest.mark.parametrize("B,S,E,H", [(2, 7, 64, 2), (1, 33, 128, 2), (2, 100, 256, 4), (1, 45, 96, 2),
                                     (1, 600, 128, 2), (2, 64, 512, 4)])
def test_legacy_matches_reference_hip_kernels(dev, B, S, E, H):
    """Same device input through the reference's own launcher (its flash
    kernel for D in {32,64} and S <= 512, else its fallback)."""
    ref = _ref_or_skip()
    qkv = O.seeded_planar(99 + S, B, S, E)
    d_qkv = dev_t(qkv)
    r_out = torch.zeros((B * S, E), device=dev)
    r_p = torch.zeros((B, H, S, S), device=dev)
    ref.launch(d_qkv.data_ptr(), r_out.data_ptr(), r_p.data_ptr(), B, S, E, H)
    o_out = torch.zeros((B * S, E), device=dev)
    o_p = torch.zeros((B, H, S, S), device=dev)
    A.launch_multihead_attention(d_qkv, o_out, o_p, B, S, E, H)
    ro, rp = host(r_out), host(r_p)
    assert np.abs(host(o_out) - ro).max() <= TOL_O
    assert np.abs(host(o_p) - rp).max() <= TOL_P
    # and the oracle agrees with the reference kernels on the same input
    want_o, want_p = O.launch_multihead_attention(qkv, B, S, E, H)
    assert np.abs(want_o - ro).max() <= 2e-6
    assert np.abs(want_p - rp).max() <= 1e-6


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,Sq,Sk,H,D", [(2, 40, 40, 3, 64), (1, 17, 90, 2, 32), (2, 64, 200, 2, 128),
                                         (1, 33, 33, 2, 48), (1, 3, 70, 2, 256), (1, 20, 150, 2, 64),
                                         (2, 200, 256, 2, 64)])
def test_strided_interleaved_layout(dev, B, Sq, Sk, H, D, causal):
    """q, k, v as views into the caller's row-interleaved [T, 3E] buffer
    (src/transformer_layer.cpp:217) -- the layout the stride-aware API takes
    without a repack; Sq < Sk exercises the bottom-right causal offset."""
    E = H * D
    kbuf = O.fill_normal(Sk * 7 + D, B * Sk * 3 * E).reshape(B, Sk, 3, H, D)
    qbuf = O.fill_normal(Sq * 5 + D, B * Sq * 3 * E).reshape(B, Sq, 3, H, D)
    q, k, v = qbuf[:, :, 0], kbuf[:, :, 1], kbuf[:, :, 2]
    want_o, want_p = O.attention(q, k, v, causal=causal, want_probs=True)
    dq, dk = dev_t(qbuf), dev_t(kbuf)
    probs = torch.empty((B, H, Sq, Sk), device=dev)
    out = A.attention(dq[:, :, 0], dk[:, :, 1], dk[:, :, 2], probs=probs, causal=causal)
    assert np.abs(host(out) - want_o).max() <= TOL_O
    assert np.abs(host(probs) - want_p).max() <= TOL_P
    out2 = A.attention(dq[:, :, 0], dk[:, :, 1], dk[:, :, 2], causal=causal)
    assert np.abs(host(out2) - want_o).max() <= TOL_O


@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("kv,splits", [(1, 1), (50, 1), (777, None), (777, 5), (2048, 16), (300, 64)])
def test_decode_matches_last_row(dev, D, kv, splits):
    B, H = 3, 4
    q, k, v = O.seeded_bshd(kv * 3 + D, B, 1, kv, H, D)
    want, _ = O.attention(q, k, v, causal=False)
    got = A.decode(dev_t(q), dev_t(k), dev_t(v), num_splits=splits)
    assert np.abs(host(got) - want).max() <= TOL_O
    # the decode row is the last row of causal self-attention over the keys
    full_q = np.concatenate([k[:, :-1], q], axis=1)  # any rows before the last
    want_last, _ = O.attention(full_q, k, v, causal=True)
    assert np.abs(host(got) - want_last[:, -1:]).max() <= TOL_O


def test_decode_split_count_independent(dev):
    B, H, kv, D = 4, 6, 1500, 64
    q, k, v = (dev_t(x) for x in O.seeded_bshd(5, B, 1, kv, H, D))
    base = host(A.decode(q, k, v, num_splits=1))
    for ns in (2, 3, 7, 16, 64):
        assert np.abs(host(A.decode(q, k, v, num_splits=ns)) - base).max() <= 5e-6


# ---------------------------------------------------------------- BASELINE configs
# Whole-tensor parity at every BASELINE config is in tests/test_fullsize_gpu.py.
CONFIGS = {  # name: (B, H, S, D)
    "c1": (32, 8, 256, 32),
    "c2": (32, 8, 256, 64),
    "c3": (8, 12, 1024, 64),
    "c4": (4, 16, 2048, 128),
}


def test_constant_v_and_zero_k_full_size(dev):
    """Closed-form answers at the c3 shape: constant V -> O = that constant;
    K = 0 -> causal O is the prefix mean of V."""
    B, H, S, D = CONFIGS["c3"]
    q = torch.randn(B, S, H, D, device=dev)
    k = torch.zeros(B, S, H, D, device=dev)
    v = torch.randn(B, S, H, D, device=dev)
    out = A.attention(q, k, v, causal=True)
    prefix = v.double().cumsum(1) / torch.arange(1, S + 1, device=dev, dtype=torch.float64)[None, :, None, None]
    assert (out.double() - prefix).abs().max().item() <= 1e-4
    vc = torch.full_like(v, -1.25)
    out = A.attention(q, torch.randn_like(q), vc, causal=True)
    assert (out + 1.25).abs().max().item() <= 1e-5


# ---------------------------------------------------------------- bf16 variant
TOL_BF16 = 2e-2


def _bf16_inputs(seed, B, Sq, Sk, H, D):
    q, k, v = O.seeded_bshd(seed, B, Sq, Sk, H, D)
    tq, tk, tv = (dev_t(x).to(torch.bfloat16) for x in (q, k, v))
    # the exact (bf16-representable) values the kernel reads, as fp32
    rq, rk, rv = (t.float().cpu().numpy() for t in (tq, tk, tv))
    assert np.array_equal(rq, O.round_bf16(q))  # torch and the oracle round alike (RNE)
    return (q, k, v), (tq, tk, tv), (rq, rk, rv)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("with_probs", [False, True])
@pytest.mark.parametrize("B,Sq,Sk,H,D", [(2, 40, 40, 3, 64), (1, 130, 130, 2, 32), (2, 64, 64, 2, 128),
                                         (1, 17, 90, 2, 64), (1, 1, 33, 1, 32)])
def test_bf16_matches_f64_on_rounded_inputs(dev, B, Sq, Sk, H, D, causal, with_probs):
    (q, k, v), (tq, tk, tv), (rq, rk, rv) = _bf16_inputs(Sq * 7 + D, B, Sq, Sk, H, D)
    want, want_p = O.attention(rq, rk, rv, causal=causal, want_probs=True, f64=True)
    probs = torch.empty((B, H, Sq, Sk), device=dev) if with_probs else None
    got = host(A.attention(tq, tk, tv, probs=probs, causal=causal))
    assert np.isfinite(got).all()
    assert np.abs(got - want).max() <= TOL_BF16
    if with_probs:
        # P is computed from bf16 inputs with fp32 accumulation: near-exact
        assert np.abs(host(probs) - want_p).max() <= 1e-5
    # distance to the unrounded fp32 problem is reported by the bench; here
    # only sanity-bounded
    full, _ = O.attention(q, k, v, causal=causal)
    assert np.abs(got - full).max() <= 0.1


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,Sq,Sk,H,D", [(1, 300, 300, 2, 64), (2, 129, 129, 3, 32), (1, 50, 200, 2, 64),
                                         (1, 257, 1000, 1, 64), (3, 128, 128, 2, 32), (1, 33, 33, 1, 64),
                                         (1, 1, 1, 1, 64), (2, 500, 520, 2, 32)])
def test_bf16_more_shapes(dev, B, Sq, Sk, H, D, causal):
    """bf16 without probs at D = 32 / 64: several 128-query blocks, ragged
    Sq / Sk, Sq != Sk (causal bottom-right offset), a single row; against
    float64 on the bf16-rounded inputs."""
    (q, k, v), (tq, tk, tv), (rq, rk, rv) = _bf16_inputs(Sq * 11 + Sk + D, B, Sq, Sk, H, D)
    want, _ = O.attention(rq, rk, rv, causal=causal, f64=True)
    got = host(A.attention(tq, tk, tv, causal=causal))
    assert np.isfinite(got).all()
    assert np.abs(got - want).max() <= TOL_BF16


# ---------------------------------------------------------------- unfused helpers
# Row kernels (D = 32/64/128, aligned): S on and off the 32-row tile grid, the
# register-resident softmax at 256/512/1024/2048 columns and the sweep softmax
# beyond; keys split over workgroups (few sequences) and the grouped weighted
# sum (>= 256 query groups, spare waves when S/32 is not a multiple of 4);
# per-element kernels: other D, S % 4 != 0 (weighted sum).
@pytest.mark.parametrize("B,S,D", [(1, 1, 8), (2, 33, 32), (1, 70, 48), (3, 64, 64), (2, 45, 128),
                                   (1, 20, 160), (32, 256, 32), (2, 100, 64), (1, 36, 128), (1, 30, 32),
                                   (2, 500, 32), (1, 1024, 64), (1, 2048, 128), (1, 2052, 32),
                                   (256, 64, 32), (256, 70, 64), (256, 36, 128)])
def test_unfused_helpers_match_oracle_and_reference(dev, B, S, D):
    """launch_scaled_dot_product / launch_softmax / launch_attention_weighted_sum
    (include/hip_kernels.h:44-46) against the oracle and, where the reference
    build is present, the reference's own kernels on the same device buffers."""
    x = O.fill_normal(B * 31 + S * 7 + D, 3 * B * S * D).reshape(3, B * S, D)
    dq, dk, dv = (dev_t(a) for a in x)
    scores = torch.full((B * S, S), float("nan"), device=dev)
    probs = torch.full((B * S, S), float("nan"), device=dev)
    out = torch.full((B * S, D), float("nan"), device=dev)
    A.launch_scaled_dot_product(dq, dk, scores, B, S, D)
    A.launch_softmax(scores, probs, B, S)
    A.launch_attention_weighted_sum(probs, dv, out, B, S, D)
    ws = O.scaled_dot_product(x[0], x[1], B, S, D)
    assert np.abs(host(scores) - ws).max() <= 1e-4
    wp = O.softmax_rows(host(scores), B, S)  # same input as the GPU softmax saw
    assert np.abs(host(probs) - wp).max() <= TOL_P
    wo = O.attention_weighted_sum(host(probs), x[2], B, S, D)
    assert np.abs(host(out) - wo).max() <= TOL_O
    if O.ref_available():
        ref = O.ref_lib()
        rs = torch.zeros_like(scores)
        rp = torch.zeros_like(probs)
        ro = torch.zeros_like(out)
        ref.sdp(dq.data_ptr(), dk.data_ptr(), rs.data_ptr(), B, S, D)
        ref.softmax(scores.data_ptr(), rp.data_ptr(), B, S)
        ref.wsum(probs.data_ptr(), dv.data_ptr(), ro.data_ptr(), B, S, D)
        assert np.abs(host(scores) - host(rs)).max() <= 1e-4
        assert np.abs(host(probs) - host(rp)).max() <= TOL_P
        assert np.abs(host(out) - host(ro)).max() <= TOL_O


def test_unfused_helpers_unaligned_views(dev):
    """Buffers one float off 16-byte alignment take the per-element / sweep
    kernels; results match the oracle as on aligned buffers."""
    B, S, D = 2, 64, 32
    x = O.fill_normal(4242, 3 * B * S * D).reshape(3, B * S, D)
    flat = [torch.zeros(B * S * D + 1, device=dev) for _ in range(3)]
    for t, a in zip(flat, x):
        t[1:] = torch.from_numpy(a.reshape(-1)).to(dev)
    dq, dk, dv = (t[1:] for t in flat)
    sbuf = torch.full((B * S * S + 1,), float("nan"), device=dev)
    pbuf = torch.full((B * S * S + 1,), float("nan"), device=dev)
    obuf = torch.full((B * S * D + 1,), float("nan"), device=dev)
    scores, probs, out = sbuf[1:], pbuf[1:], obuf[1:]
    A.launch_scaled_dot_product(dq, dk, scores, B, S, D)
    A.launch_softmax(scores, probs, B, S)
    A.launch_attention_weighted_sum(probs, dv, out, B, S, D)
    ws = O.scaled_dot_product(x[0], x[1], B, S, D)
    assert np.abs(host(scores).reshape(B * S, S) - ws).max() <= 1e-4
    wp = O.softmax_rows(host(scores).reshape(B * S, S), B, S)
    assert np.abs(host(probs).reshape(B * S, S) - wp).max() <= TOL_P
    wo = O.attention_weighted_sum(host(probs).reshape(B * S, S), x[2], B, S, D)
    assert np.abs(host(out).reshape(B * S, D) - wo).max() <= TOL_O


# Head dims above 128 with D % 4 == 0 up to 512 run the head-dim-split MFMA
# kernel (fa_wide.hip; 64 dims per wave, four waves per 32 queries padded to
# 256, eight padded to 512); other D above 128 the one-wave-per-row kernel
# (generic.hip).  S below, across and
# off the 32-row tile, several query blocks per (b, h), Sq < Sk.
WIDE_FWD = [
    (2, 33, 33, 2, 132), (1, 1, 1, 2, 256), (1, 70, 70, 3, 160), (2, 130, 130, 2, 192), (1, 257, 257, 1, 256),
    (1, 100, 100, 2, 200), (2, 40, 90, 2, 256), (1, 300, 300, 1, 228), (1, 64, 64, 2, 150), (1, 9, 40, 2, 260),
    (1, 70, 70, 2, 512), (2, 33, 100, 1, 384), (1, 130, 130, 1, 300), (1, 1, 1, 1, 512), (1, 40, 40, 1, 520),
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,Sq,Sk,H,D", WIDE_FWD)
def test_wide_head_dim_forward_matches_oracle(dev, B, Sq, Sk, H, D, causal):
    """[B, S, H, D] views with probs (NaN directly after the probs in the same
    allocation: a store past the last row would be visible as a changed
    value; every probability written) and without, against the oracle."""
    q, k, v = O.seeded_bshd(D * 31 + Sq + Sk, B, Sq, Sk, H, D)
    want_o, want_p = O.attention(q, k, v, causal=causal, want_probs=True)
    dq, dk, dv = dev_t(q), dev_t(k), dev_t(v)
    n = B * H * Sq * Sk
    pbuf = torch.full((n + 4096,), float("nan"), device=dev)
    probs = pbuf[:n].view(B, H, Sq, Sk)
    out = A.attention(dq, dk, dv, probs=probs, causal=causal)
    got_p = host(pbuf)
    assert np.isnan(got_p[n:]).all()
    assert np.isfinite(got_p[:n]).all()
    assert np.abs(host(out) - want_o).max() <= TOL_O
    assert np.abs(got_p[:n].reshape(B, H, Sq, Sk) - want_p).max() <= TOL_P
    out2 = A.attention(dq, dk, dv, causal=causal)
    assert np.abs(host(out2) - want_o).max() <= TOL_O


@pytest.mark.parametrize("B,S,E,H", [(2, 130, 512, 2), (1, 300, 640, 4), (1, 77, 1024, 4), (1, 100, 1024, 2)])
def test_wide_head_dim_dropin_matches_reference_launcher(dev, B, S, E, H):
    """HipGPT's call at D = 256, 160, 256, 512: against the reference's launcher
    (its fallback kernel) on the same device buffers, with and without probs."""
    ref = _ref_or_skip()
    qkv = O.seeded_planar(171 + S + E, B, S, E)
    d_qkv = dev_t(qkv)
    r_out = torch.zeros((B * S, E), device=dev)
    r_p = torch.zeros((B, H, S, S), device=dev)
    ref.launch(d_qkv.data_ptr(), r_out.data_ptr(), r_p.data_ptr(), B, S, E, H)
    o_out = torch.full((B * S, E), float("nan"), device=dev)
    o_p = torch.full((B, H, S, S), float("nan"), device=dev)
    A.launch_multihead_attention(d_qkv, o_out, o_p, B, S, E, H)
    assert np.abs(host(o_out) - host(r_out)).max() <= TOL_O
    assert np.abs(host(o_p) - host(r_p)).max() <= TOL_P
    o2 = torch.full((B * S, E), float("nan"), device=dev)
    A.launch_multihead_attention(d_qkv, o2, None, B, S, E, H)
    assert np.abs(host(o2) - host(r_out)).max() <= TOL_O
