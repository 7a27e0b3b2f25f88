"""CPU tests that pin the oracle (oracle/attn_oracle.c) before it is trusted.

Each check is chosen so that a plausible slip in the restatement (dropped
scale, wrong stride, transposed operand, off-by-one causal limit, missing
max subtraction) fails at least one of them: closed-form invariants,
numpy brute force on tiny inputs, the published SplitMix64 vector, and the
golden vectors produced by the reference's own HIP kernels.
"""
import glob
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def np_attention(q, k, v, causal):
    """Brute force with numpy in float64 (explicit mask, explicit softmax)."""
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    qd, kd, vd = (x.astype(np.float64) for x in (q, k, v))
    s = np.einsum("bihd,bjhd->bhij", qd, kd) / np.sqrt(D)
    if causal:
        off = Sk - Sq
        mask = np.arange(Sk)[None, :] > (np.arange(Sq)[:, None] + off)
        s = np.where(mask[None, None], -np.inf, s)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    o = np.einsum("bhij,bjhd->bihd", p, vd)
    return o, p


def test_splitmix64_published_vector():
    # Test vector of the SplitMix64 reference implementation, seed 1234567.
    assert O.splitmix64(1234567, 5) == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821,
    ]


def test_fill_normal_moments_and_determinism():
    x = O.fill_normal(0x48495047, 2_000_000)
    assert abs(float(x.mean())) < 3e-3
    assert abs(float(x.std()) - 1.0) < 3e-3
    assert abs(float((x.astype(np.float64) ** 4).mean()) - 3.0) < 0.03  # Gaussian kurtosis
    assert np.array_equal(x[:1000], O.fill_normal(0x48495047, 1000))
    assert not np.array_equal(x[:1000], O.fill_normal(0x48495048, 1000))


def test_round_bf16_rne():
    vals = np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 1.0 + 2**-9, -2.5, 3.0e38], dtype=np.float32)
    r = O.round_bf16(vals)
    # 1+2^-8 is a tie -> even (1.0); 1+3*2^-8 tie -> up to 1+2^-6; 1+2^-9 rounds down
    assert r[0] == 1.0 and r[1] == 1.0 and r[2] == np.float32(1.0 + 2**-6) and r[3] == 1.0
    assert r[4] == -2.5
    bits = r.view(np.uint32)
    assert np.all(bits & 0xFFFF == 0)


@pytest.mark.parametrize("variant", [O.FLASH, O.FALLBACK])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,Sq,Sk,H,D", [(1, 1, 1, 1, 32), (2, 7, 7, 2, 32), (1, 33, 33, 2, 64),
                                         (2, 31, 31, 1, 48), (1, 5, 12, 2, 16), (1, 64, 64, 1, 128)])
def test_restatement_matches_bruteforce(variant, causal, B, Sq, Sk, H, D):
    q, k, v = O.seeded_bshd(B * 1000 + Sq * 10 + D, B, Sq, Sk, H, D)
    o, p = O.attention(q, k, v, causal=causal, variant=variant, want_probs=True)
    o64, p64 = np_attention(q, k, v, causal)
    assert np.abs(o - o64).max() < 2e-6
    assert np.abs(p - p64).max() < 1e-6
    of, pf = O.attention(q, k, v, causal=causal, want_probs=True, f64=True)
    assert np.abs(of - o64).max() < 1e-6
    assert np.abs(pf - p64).max() < 1e-7


@pytest.mark.parametrize("variant", [O.FLASH, O.FALLBACK])
def test_invariants(variant):
    B, S, H, D = 2, 40, 2, 32
    q, k, v = O.seeded_bshd(11, B, S, S, H, D)
    # constant V -> O is that constant
    vc = np.full_like(v, 0.75)
    o, _ = O.attention(q, k, vc, causal=True, variant=variant)
    assert np.abs(o - 0.75).max() < 1e-6
    # K = 0 -> uniform P: 1/S non-causal, 1/(i+1) causal; O = (prefix) mean of V
    kz = np.zeros_like(k)
    o, p = O.attention(q, kz, v, causal=False, variant=variant, want_probs=True)
    assert np.abs(p - 1.0 / S).max() < 1e-7
    assert np.abs(o - v.mean(axis=1, keepdims=True)).max() < 1e-5
    o, p = O.attention(q, kz, v, causal=True, variant=variant, want_probs=True)
    i = np.arange(S)
    exp_p = np.where(i[None, :] <= i[:, None], 1.0 / (i[:, None] + 1), 0.0)
    assert np.abs(p - exp_p[None, None]).max() < 1e-7
    prefix_mean = np.cumsum(v.astype(np.float64), axis=1) / (i[None, :, None, None] + 1)
    assert np.abs(o - prefix_mean).max() < 1e-5
    # causal row 0 -> V_0
    o, _ = O.attention(q, k, v, causal=True, variant=variant)
    assert np.abs(o[:, 0] - v[:, 0]).max() == 0.0
    # last row: causal == non-causal
    onc, _ = O.attention(q, k, v, causal=False, variant=variant)
    assert np.abs(o[:, -1] - onc[:, -1]).max() == 0.0
    # S = 1 -> O = V
    o1, _ = O.attention(q[:, :1].copy(), k[:, :1].copy(), v[:, :1].copy(), variant=variant)
    assert np.abs(o1 - v[:, :1]).max() == 0.0
    # rows sum to one, causal P zero above the diagonal
    _, p = O.attention(q, k, v, causal=True, variant=variant, want_probs=True)
    assert np.abs(p.sum(-1) - 1).max() < 1e-5
    assert np.all(p[..., np.triu_indices(S, 1)[0], np.triu_indices(S, 1)[1]] == 0)
    # non-causal O invariant under a key/value permutation
    perm = np.random.default_rng(0).permutation(S)
    o_a, _ = O.attention(q, k, v, variant=variant)
    o_b, _ = O.attention(q, k[:, perm].copy(), v[:, perm].copy(), variant=variant)
    assert np.abs(o_a - o_b).max() < 2e-6
    # huge scores -> O = V[argmax] with no NaN/inf
    qh = q * 1e4
    oh, _ = O.attention(qh, k, v, variant=variant)
    s = np.einsum("bihd,bjhd->bhij", qh.astype(np.float64), k.astype(np.float64))
    am = s.argmax(-1)  # [B,H,S]
    want = np.take_along_axis(v.transpose(0, 2, 1, 3), am[..., None], axis=2).transpose(0, 2, 1, 3)
    assert np.isfinite(oh).all()
    assert np.abs(oh - want).max() < 1e-5


def test_planar_launcher_mirror_and_bad_config():
    B, S, E, H = 2, 20, 64, 2
    qkv = O.seeded_planar(5, B, S, E)
    out, probs = O.launch_multihead_attention(qkv, B, S, E, H)
    q, k, v = O.planar_qkv(qkv, B, S, E, H)
    o64, p64 = np_attention(q, k, v, False)
    assert np.abs(out.reshape(B, S, H, E // H) - o64).max() < 2e-6
    assert np.abs(probs - p64).max() < 1e-6
    with pytest.raises(ValueError, match="Bad MHA config"):
        O.launch_multihead_attention(qkv, B, S, 63, 2)
    with pytest.raises(ValueError, match="Bad MHA config"):
        O.launch_multihead_attention(qkv, B, S, E, 0)


def test_pairs_subset_matches_full():
    q, k, v = O.seeded_bshd(3, 3, 24, 24, 4, 32)
    full, _ = O.attention(q, k, v, causal=True)
    part, _ = O.attention(q, k, v, causal=True, pairs=[(1, 2), (2, 0)])
    assert np.array_equal(part[1, :, 2], full[1, :, 2])
    assert np.array_equal(part[2, :, 0], full[2, :, 0])
    assert np.all(part[0] == 0)


def _golden_files():
    return sorted(glob.glob(os.path.join(GOLDEN, "ref_*.npz")))


@pytest.mark.skipif(not _golden_files(), reason="no golden vectors generated yet")
@pytest.mark.parametrize("path", _golden_files(), ids=os.path.basename)
def test_oracle_matches_reference_golden(path):
    """Golden vectors written by the reference's own HIP launcher
    (tests/golden/make_golden.py on an MI355X): same planar input regenerated
    from the seed, oracle compared with the reference's O and P."""
    g = np.load(path, allow_pickle=False)
    B, S, E, H, seed = (int(g[n]) for n in ("B", "S", "E", "H", "seed"))
    qkv = O.seeded_planar(seed, B, S, E)
    assert np.float32(qkv.astype(np.float64).sum()) == np.float32(g["qkv_sum"])
    out, probs = O.launch_multihead_attention(qkv, B, S, E, H)
    assert np.abs(out - g["out"].reshape(out.shape)).max() < 2e-6
    rows = g["prob_rows"]
    assert np.abs(probs[:, :, rows, :] - g["probs"]).max() < 1e-6


@pytest.mark.parametrize("B,S,D", [(1, 1, 8), (2, 33, 32), (1, 70, 48), (3, 17, 64)])
def test_unfused_helpers_match_bruteforce(B, S, D):
    """scaled_dot_product / softmax / weighted_sum restatements
    (src/hip_kernels.cpp:454-532) against numpy in float64."""
    x = O.fill_normal(B * 100 + S + D, 3 * B * S * D).reshape(3, B * S, D)
    s = O.scaled_dot_product(x[0], x[1], B, S, D)
    q, k, v = (a.reshape(B, S, D).astype(np.float64) for a in x)
    ref = (np.einsum("bid,bjd->bij", q, k) / np.sqrt(D)).reshape(B * S, S)
    assert np.abs(s - ref).max() < 2e-6
    p = O.softmax_rows(s, B, S)
    e = np.exp(ref - ref.max(-1, keepdims=True))
    e /= e.sum(-1, keepdims=True)
    assert np.abs(p - e).max() < 1e-6
    assert np.abs(p.sum(-1) - 1).max() < 1e-5
    o = O.attention_weighted_sum(p, x[2], B, S, D)
    ro = np.einsum("bij,bjd->bid", e.reshape(B, S, S), v).reshape(B * S, D)
    assert np.abs(o - ro).max() < 2e-6
    # composition equals the fused restatement (H = 1, planar layout)
    qkv = np.concatenate([x[0].ravel(), x[1].ravel(), x[2].ravel()])
    fused, probs = O.launch_multihead_attention(qkv, B, S, D, 1)
    assert np.abs(fused - o).max() < 2e-6
    assert np.abs(probs.reshape(B * S, S) - p).max() < 1e-6


def _np_planar_forward(qkv, B, S, E, H, causal):
    q, k, v = (x.astype(np.float64) for x in O.planar_qkv(qkv, B, S, E, H))
    o, p = np_attention(q, k, v, causal)
    return o.reshape(B * S, E), p


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,S,E,H", [(1, 5, 8, 2), (2, 4, 6, 1), (1, 7, 12, 3)])
def test_backward_restatement_matches_finite_differences(B, S, E, H, causal):
    """oracle_mha_backward (src/hip_kernels.cpp:1159-1272) against central
    differences of L = sum(dO * O(qkv)) computed in float64 brute force.  Every
    planar element is perturbed, so a dropped Dq term, a missing scale, a swapped
    dK/dV plane or a transposed probs index each fail.  With causal probs the
    unmasked formula must give the causal gradient (P = 0 above the diagonal)."""
    qkv = O.seeded_planar(B * 100 + S * 10 + E + int(causal), B, S, E)
    go = O.fill_normal(7 + S, B * S * E).reshape(B * S, E)
    _, p64 = _np_planar_forward(qkv, B, S, E, H, causal)
    got = O.mha_backward(go, qkv, p64.astype(np.float32), B, S, E, H)
    x = qkv.astype(np.float64)
    num = np.zeros_like(x)
    eps = 1e-5
    for n in range(x.size):
        xp = x.copy()
        xp[n] += eps
        lp = (go * _np_planar_forward(xp, B, S, E, H, causal)[0]).sum()
        xp[n] -= 2 * eps
        lm = (go * _np_planar_forward(xp, B, S, E, H, causal)[0]).sum()
        num[n] = (lp - lm) / (2 * eps)
    assert np.abs(got - num).max() < 2e-5 * max(1.0, np.abs(num).max())
    with pytest.raises(ValueError, match="Bad MHA config"):
        O.mha_backward(go, qkv, p64.astype(np.float32), B, S, E, 0)


def test_backward_restatement_threads_give_identical_results():
    """oracle_mha_backward_mt: (b, h) pairs on several host threads write
    disjoint elements, so the result equals the one-thread restatement bit
    for bit."""
    B, S, E, H = 3, 37, 96, 4
    qkv = O.seeded_planar(77, B, S, E)
    go = O.fill_normal(78, B * S * E)
    _, p = O.launch_multihead_attention(qkv, B, S, E, H, causal=True, want_probs=True)
    one = O.mha_backward(go, qkv, p, B, S, E, H)
    for nt in (2, 5, 64):
        assert np.array_equal(O.mha_backward(go, qkv, p, B, S, E, H, nthreads=nt), one)
