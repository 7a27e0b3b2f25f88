"""GPU test of hipgpt_attn_bwd_qkv_planar_noalloc (include/hipgpt_attn.h): the
backward for callers that cannot allocate, whose row-dot workspace is a
fixed per-device array inside the library.  Called through the C ABI and
compared with hipgpt_attn_bwd_qkv_planar (caller workspace) on the same
buffers: the same kernels run, so the gradients must agree bit for bit.  Two
calls in a row, the second on a smaller problem (the array keeps the first
call's contents), in both masking modes and on each backward path that uses
the workspace (D = 64 tiled kernels, D = 128 and D = 16 global-memory
kernels); a problem beyond the array is rejected before any launch.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hipgpt_amd import _lib

pytestmark = pytest.mark.gpu


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _problem(B, S, E, H, causal, seed, dev):
    qkv = O.seeded_planar(seed + B * 7919 + S * 31 + E, B, S, E)
    go = O.fill_normal(seed + 99 + S + E, B * S * E)
    _, probs = O.launch_multihead_attention(qkv, B, S, E, H, causal=causal, want_probs=True)
    return (torch.from_numpy(qkv).to(dev), torch.from_numpy(go).to(dev), torch.from_numpy(probs).to(dev))


def _both(L, B, S, E, H, causal, seed, dev):
    qkv, go, probs = _problem(B, S, E, H, causal, seed, dev)
    ws = torch.empty(L.hipgpt_attn_bwd_workspace_bytes(B, S, H) // 4, device=dev)
    want = torch.full((3 * B * S * E,), float("nan"), device=dev)
    got = torch.full_like(want, float("nan"))
    stream = torch.cuda.current_stream().cuda_stream
    rc = L.hipgpt_attn_bwd_qkv_planar(_ptr(go), _ptr(qkv), _ptr(probs), _ptr(want), B, S, E, H, int(causal),
                                      _ptr(ws), ws.numel() * 4, stream)
    assert rc == _lib.OK
    rc = L.hipgpt_attn_bwd_qkv_planar_noalloc(_ptr(go), _ptr(qkv), _ptr(probs), _ptr(got), B, S, E, H,
                                              int(causal), stream)
    assert rc == _lib.OK
    torch.cuda.synchronize()
    return want.cpu().numpy(), got.cpu().numpy()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("first,second", [((4, 512, 512, 8), (2, 130, 256, 4)),    # D = 64, tiled kernels
                                          ((2, 300, 512, 4), (1, 77, 256, 2)),     # D = 128, global kernels
                                          ((3, 96, 64, 4), (1, 33, 32, 2))])       # D = 16, global kernels
def test_noalloc_backward_matches_workspace_entry(dev, first, second, causal):
    L = _lib.lib()
    for i, (B, S, E, H) in enumerate((first, second)):
        want, got = _both(L, B, S, E, H, causal, 17 + i, dev)
        assert np.isfinite(got).all()
        assert np.array_equal(got, want), (B, S, E, H)


def test_noalloc_backward_rejects_problems_beyond_its_scratch(dev):
    """B*H*S = 2^21 > 2^20 floats of scratch: rejected on the host before the
    pointers are looked at, so the call passes null pointers and can never
    launch anything."""
    L = _lib.lib()
    rc = L.hipgpt_attn_bwd_qkv_planar_noalloc(None, None, None, None, 64, 2048, 2048, 16, 0, None)
    assert rc == _lib.ERR_SCRATCH
    assert b"scratch" in L.hipgpt_attn_strerror(rc)
    # within the limit, the null pointers are what is rejected
    rc = L.hipgpt_attn_bwd_qkv_planar_noalloc(None, None, None, None, 1, 64, 64, 2, 0, None)
    assert rc == _lib.ERR_INVALID


@pytest.mark.parametrize("B,S,E,H", [(4, 512, 512, 8),    # D = 64: tiled kernels, scratch used
                                     (2, 300, 512, 4)])   # D = 128: scratch used
def test_noalloc_backward_under_graph_capture(dev, B, S, E, H):
    """The noalloc call captured into a HIP graph (after one eager call, which
    looks up the scratch address and sets kernel attributes): every replay,
    with eager calls of both entry points in between, equals the caller-
    workspace entry point bit for bit."""
    L = _lib.lib()
    qkv, go, probs = _problem(B, S, E, H, True, 23, dev)
    ws = torch.empty(L.hipgpt_attn_bwd_workspace_bytes(B, S, H) // 4, device=dev)
    want = torch.full((3 * B * S * E,), float("nan"), device=dev)
    got = torch.full_like(want, float("nan"))

    def workspace_call():
        rc = L.hipgpt_attn_bwd_qkv_planar(_ptr(go), _ptr(qkv), _ptr(probs), _ptr(want), B, S, E, H, 1,
                                          _ptr(ws), ws.numel() * 4, torch.cuda.current_stream().cuda_stream)
        assert rc == _lib.OK

    def noalloc_call():
        rc = L.hipgpt_attn_bwd_qkv_planar_noalloc(_ptr(go), _ptr(qkv), _ptr(probs), _ptr(got), B, S, E, H, 1,
                                                  torch.cuda.current_stream().cuda_stream)
        assert rc == _lib.OK

    workspace_call()
    noalloc_call()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        noalloc_call()
    torch.cuda.synchronize()
    for k in range(3):
        got.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {k} differs"
        workspace_call()
        noalloc_call()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"eager calls after replay {k} differ"
