"""GPU tests of the KV-cached decode step (hipgpt_attn_decode_kvcache): the
step HipGPT's generation loop (src/gpt_model.cpp:261-273) would take instead
of recomputing the whole window per token.

Oracle: the reference semantics of a decode row is the last row of full
attention over the visible keys (src/hip_kernels.cpp:329-402 at S = kv_len),
i.e. the oracle's restatement over the cached rows plus the new one.  The
cache rows past each sequence's length are filled with NaN, so reading any of
them would poison the output.  Bar: fp32 max-abs 1e-4.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hipgpt_amd import attention as A

pytestmark = pytest.mark.gpu

TOL_O = 1e-4


def dev_t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def oracle_row(q, keys, vals):
    """q [H, D], keys/vals [n, H, D] -> [H, D] (reference fallback arithmetic)."""
    out, _ = O.attention(q[None, None], keys[None], vals[None], causal=False, variant=O.FALLBACK)
    return out[0, 0]


def make_cache(seed, B, max_len, H, D, lens):
    x = O.fill_normal(seed, 2 * B * max_len * H * D).reshape(2, B, max_len, H, D)
    kc, vc = x[0].copy(), x[1].copy()
    for b, n in enumerate(lens):
        if 0 <= n < max_len:
            kc[b, n:] = np.nan
            vc[b, n:] = np.nan
    return kc, vc


@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("splits", [1, None, 7])
def test_step_matches_oracle_and_appends(dev, D, splits):
    B, H, max_len = 5, 3, 300
    lens_h = np.array([0, 1, 17, 128, 299], dtype=np.int32)
    kc, vc = make_cache(D + 11, B, max_len, H, D, lens_h)
    q, kn, vn = O.fill_normal(D * 7 + 1, 3 * B * H * D).reshape(3, B, H, D)
    d_kc, d_vc, lens = dev_t(kc), dev_t(vc), dev_t(lens_h)
    got = host(A.decode_kvcache(dev_t(q), dev_t(kn), dev_t(vn), d_kc, d_vc, lens, num_splits=splits))
    assert np.isfinite(got).all()
    for b, n in enumerate(lens_h):
        keys = np.concatenate([kc[b, :n], kn[b][None]], axis=0)
        vals = np.concatenate([vc[b, :n], vn[b][None]], axis=0)
        assert np.abs(got[b] - oracle_row(q[b], keys, vals)).max() <= TOL_O, b
    nkc, nvc = host(d_kc), host(d_vc)
    for b, n in enumerate(lens_h):
        assert np.array_equal(nkc[b, :n], kc[b, :n]) and np.array_equal(nvc[b, :n], vc[b, :n])
        assert np.array_equal(nkc[b, n], kn[b]) and np.array_equal(nvc[b, n], vn[b])
        assert np.isnan(nkc[b, n + 1:]).all() and np.isnan(nvc[b, n + 1:]).all()
    assert np.array_equal(host(lens), lens_h + 1)


def test_full_or_invalid_length_is_nan_and_untouched(dev):
    B, H, D, max_len = 3, 2, 64, 40
    lens_h = np.array([max_len, -1, 3], dtype=np.int32)
    kc, vc = make_cache(3, B, max_len, H, D, lens_h)
    q, kn, vn = O.fill_normal(4, 3 * B * H * D).reshape(3, B, H, D)
    for splits in (1, 4):
        d_kc, d_vc, lens = dev_t(kc), dev_t(vc), dev_t(lens_h)
        got = host(A.decode_kvcache(dev_t(q), dev_t(kn), dev_t(vn), d_kc, d_vc, lens, num_splits=splits))
        assert np.isnan(got[:2]).all() and np.isfinite(got[2]).all()
        assert np.array_equal(host(lens), np.array([max_len, -1, 4], dtype=np.int32))
        nkc = host(d_kc)
        assert np.array_equal(nkc[:2], kc[:2], equal_nan=True)
        assert np.array_equal(nkc[2, 3], kn[2])


def test_advance_off_keeps_lengths(dev):
    B, H, D, max_len = 2, 4, 128, 64
    lens_h = np.array([10, 63], dtype=np.int32)
    kc, vc = make_cache(9, B, max_len, H, D, lens_h)
    q, kn, vn = (dev_t(x) for x in O.fill_normal(10, 3 * B * H * D).reshape(3, B, H, D))
    lens = dev_t(lens_h)
    a = host(A.decode_kvcache(q, kn, vn, dev_t(kc), dev_t(vc), lens, advance=False))
    assert np.array_equal(host(lens), lens_h)
    b = host(A.decode_kvcache(q, kn, vn, dev_t(kc), dev_t(vc), lens, advance=True))
    assert np.array_equal(a, b)


def test_generation_loop_equals_recompute(dev):
    """Prefill caches of different lengths, then 24 steps of appending a new
    token per sequence with lengths advanced on the device: every step's
    output equals the last row of causal attention over the whole sequence
    so far, recomputed by the oracle (what HipGPT's generate loop computes
    per token without a cache)."""
    B, H, D, max_len, steps = 3, 4, 64, 96, 24
    pre = [5, 0, 40]
    kc, vc = make_cache(21, B, max_len, H, D, pre)
    d_kc, d_vc, lens = dev_t(kc), dev_t(vc), dev_t(np.array(pre, dtype=np.int32))
    seq_k = [kc[b, :n].copy() for b, n in enumerate(pre)]
    seq_v = [vc[b, :n].copy() for b, n in enumerate(pre)]
    ws = torch.empty(A.decode_workspace_bytes(B, H, D, 4) // 4, device=dev)
    for t in range(steps):
        q, kn, vn = O.fill_normal(1000 + t, 3 * B * H * D).reshape(3, B, H, D)
        got = host(A.decode_kvcache(dev_t(q), dev_t(kn), dev_t(vn), d_kc, d_vc, lens, num_splits=4, workspace=ws))
        for b in range(B):
            seq_k[b] = np.concatenate([seq_k[b], kn[b][None]], axis=0)
            seq_v[b] = np.concatenate([seq_v[b], vn[b][None]], axis=0)
            n = seq_k[b].shape[0]
            # full causal self-attention over the sequence, query rows = keys
            # except the last, which is this step's query
            full_q = np.concatenate([seq_k[b][:-1], q[b][None]], axis=0)[None]
            want, _ = O.attention(full_q, seq_k[b][None], seq_v[b][None], causal=True, variant=O.FALLBACK)
            assert np.abs(got[b] - want[0, n - 1]).max() <= TOL_O, (t, b)
    assert np.array_equal(host(lens), np.array(pre, dtype=np.int32) + steps)


def test_strided_rows_from_a_qkv_projection(dev):
    """q, k_new, v_new as column windows of one [B, 3E] projection output,
    the layout a QKV GEMM for one token per sequence produces."""
    B, H, D, max_len = 4, 3, 32, 50
    E = H * D
    lens_h = np.array([7, 0, 49, 20], dtype=np.int32)
    kc, vc = make_cache(31, B, max_len, H, D, lens_h)
    rows = dev_t(O.fill_normal(32, B * 3 * E).reshape(B, 3 * E))
    q, kn, vn = (rows[:, i * E:(i + 1) * E].view(B, H, D) for i in range(3))
    got = host(A.decode_kvcache(q, kn, vn, dev_t(kc), dev_t(vc), dev_t(lens_h)))
    r = host(rows).reshape(B, 3, H, D)
    for b, n in enumerate(lens_h):
        keys = np.concatenate([kc[b, :n], r[b, 1][None]], axis=0)
        vals = np.concatenate([vc[b, :n], r[b, 2][None]], axis=0)
        assert np.abs(got[b] - oracle_row(r[b, 0], keys, vals)).max() <= TOL_O


def test_baseline_c5_shape(dev):
    """c5 as a cache step: B=64, H=12, D=64, 2047 cached rows + the new one
    (kv_len = 2048), checked on three (b, h) pairs."""
    B, H, D, max_len = 64, 12, 64, 2048
    x = torch.randn(2, B, max_len, H, D, device=dev)
    d_kc, d_vc = x[0], x[1]
    q, kn, vn = torch.randn(3, B, H, D, device=dev)
    lens = torch.full((B,), max_len - 1, dtype=torch.int32, device=dev)
    got = host(A.decode_kvcache(q, kn, vn, d_kc, d_vc, lens))
    kc, vc = host(d_kc), host(d_vc)
    qh, knh, vnh = host(q), host(kn), host(vn)
    for b, h in [(0, 0), (17, 5), (63, 11)]:
        assert np.array_equal(kc[b, -1, h], knh[b, h])
        want = oracle_row(qh[b, h][None], kc[b, :, h][:, None], vc[b, :, h][:, None])
        assert np.abs(got[b, h] - want[0]).max() <= TOL_O
    assert np.isfinite(got).all()
