"""CPU test of the synchronisation schedule of the probs-free
one-workgroup-per-(b, h) backward (bwd_bh_kernel in hipgpt_amd/csrc/bwd_bh.h).

The kernel's waves wait on LDS flags instead of workgroup barriers: a tile's
"staged" flag and the dQ chain counter of a query tile (contributions in
descending key-tile order).  Every wait is bounded on the device, but a schedule
that could block would silently produce wrong gradients, so this test restates
each wave's sequence of waits and sets (the same key-tile assignment, job
order and flags as the kernel) and runs them under an event scheduler that
always picks one runnable wave.  It checks that every schedule completes for
every tile count 1..8, causal or not, under both a fixed and randomised
choice of the next wave.  A deadlock would leave a wave blocked with nothing
else runnable.

Restated from: key-tile assignment (sr -> kt, SIMD pairs s / nt-1-s), the
staging flags, job(): step t handles query tile kt + t (mod nt if not
causal), waiting staged[i] from the second job on; chain_add(): waits
chain[i] >= t and sets t + 1 unless last.
"""
import random

import pytest


def wave_programs(nt, causal):
    """Per wave, a list of ("wait", flag, tile, value) / ("set", flag, tile, value) ops."""
    waves = []
    for sr in range(8):
        s2 = sr >> 1
        kt = -1
        if s2 < (nt + 1) // 2:
            kt = (nt - 1 - s2 if nt - 1 - s2 > s2 else -1) if (sr & 1) else s2
        if kt < 0:
            continue
        ops = [("set", "staged", kt, 1)]
        nsteps = nt - kt if causal else nt

        def tile(k, t):
            i = k + t
            return i - nt if (not causal and i >= nt) else i

        # job t, its dQ term added one job later
        prev = None
        for t in range(nsteps):
            i = tile(kt, t)
            if t > 0:
                ops.append(("wait", "staged", i, 1))
            if prev is not None:
                ops += chain_ops(*prev, nt, causal)
            prev = (i, t)
        ops += chain_ops(*prev, nt, causal)
        waves.append((kt, ops))
    return waves


def chain_ops(i, t, nt, causal):
    nc = i + 1 if causal else nt
    ops = []
    if t > 0:
        ops.append(("wait", "chain", i, t))
    if t < nc - 1:
        ops.append(("set", "chain", i, t + 1))
    else:
        ops.append(("done", "dq", i, 0))
    return ops


def run(waves, nt, rng=None):
    flags = {}
    pos = [0] * len(waves)
    finished_dq = []
    while True:
        runnable = []
        for w, (_, ops) in enumerate(waves):
            if pos[w] >= len(ops):
                continue
            kind, flag, i, v = ops[pos[w]]
            if kind != "wait" or flags.get((flag, i), 0) >= v:
                runnable.append(w)
        if not runnable:
            break
        w = rng.choice(runnable) if rng else runnable[0]
        kind, flag, i, v = waves[w][1][pos[w]]
        if kind == "set":
            assert flags.get((flag, i), 0) == v - 1 or flag == "staged", (flag, i, v)
            flags[(flag, i)] = v
        elif kind == "done":
            finished_dq.append(i)
        pos[w] += 1
    blocked = [waves[w][0] for w in range(len(waves)) if pos[w] < len(waves[w][1])]
    return blocked, sorted(finished_dq)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("nt", range(1, 9))
def test_every_wait_ends(nt, causal):
    waves = wave_programs(nt, causal)
    assert sorted(kt for kt, _ in waves) == list(range(nt))  # each key tile owned once
    for rng in [None] + [random.Random(seed) for seed in range(20)]:
        blocked, done = run(waves, nt, rng)
        assert not blocked, f"waves of key tiles {blocked} never finish"
        assert done == list(range(nt))  # each query tile's dQ finished exactly once


def test_chain_order_is_descending_key_tiles():
    """Causal: query tile i receives its dQ terms from key tiles i, i-1, ..., 0
    in that order (the fixed summation order that makes dQ deterministic)."""
    nt = 8
    waves = wave_programs(nt, True)
    owner = {}
    for kt, ops in waves:
        for kind, flag, i, v in ops:
            if kind == "set" and flag == "chain":
                owner[(i, v)] = kt  # the contribution that raised chain[i] to v
    for i in range(nt):
        assert [owner[(i, v)] for v in range(1, i + 1)] == list(range(i, 0, -1))
