"""GPU tests: the attention kernels replayed from a captured HIP graph give the
same results as eager launches, replay after replay.

The Python entry points launch on torch's current stream, so
torch.cuda.CUDAGraph captures them.  Nothing inside a captured region
allocates or calls a torch kernel (the workspaces are passed in), and every
kernel here is deterministic (no atomics; the per-(b, h) backward sums dQ in a
fixed order), so each replay must equal the eager result bit for bit.  Eager
launches run between the replays, and the outputs are poisoned before each
replay, so a replay that wrote nothing would fail.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hipgpt_amd import attention as A

pytestmark = pytest.mark.gpu


def _replays_match_eager(run, outs, replays=3):
    run()  # eager: also sets any per-device kernel attribute before capture
    torch.cuda.synchronize()
    ref = [o.clone() for o in outs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    torch.cuda.synchronize()
    for k in range(replays):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o, r), f"replay {k} differs from the eager result"
        run()  # eager work between replays
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o, r), f"eager call after replay {k} differs"


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


@pytest.mark.parametrize("B,S,E,H", [(2, 256, 256, 8), (2, 200, 512, 8)])
def test_probs_free_pair_in_a_graph(dev, B, S, E, H):
    """Forward with lse + backward from it: D = 32 runs the one-workgroup-per-
    (b, h) backward, D = 64 the query/key-stationary pair."""
    qkv = _dev(O.seeded_planar(31 + S, B, S, E))
    go = _dev(O.fill_normal(32 + S, B * S * E))
    out = torch.empty(B * S, E, device=dev)
    lse = torch.empty(B * H * S, device=dev)
    grad = torch.empty(3 * B * S * E, device=dev)

    def run():
        A.fwd_lse_qkv_planar(qkv, out, lse, B, S, E, H, causal=True)
        A.bwd_lse_qkv_planar(go, qkv, out, lse, grad, B, S, E, H, causal=True)

    _replays_match_eager(run, [out, lse, grad])


def test_stored_probs_forward_backward_in_a_graph(dev):
    """Causal forward writing probs + the backward on them (D = 32, S = 256:
    the per-(b, h) kernel in its stored-probs mode)."""
    B, S, E, H = 2, 256, 256, 8
    qkv = _dev(O.seeded_planar(41, B, S, E))
    go = _dev(O.fill_normal(42, B * S * E))
    out = torch.empty(B * S, E, device=dev)
    probs = torch.empty(B, H, S, S, device=dev)
    grad = torch.empty(3 * B * S * E, device=dev)
    ws = torch.empty(B * H * S, device=dev)

    def run():
        A.qkv_planar(qkv, out, probs, B, S, E, H, causal=True)
        A.attention_backward(go, qkv, probs, grad, B, S, E, H, causal=True, workspace=ws)

    _replays_match_eager(run, [out, probs, grad])
