"""CPU test of the synchronisation schedule of the resident-K/V forward
(hipgpt_amd/csrc/fa_resident.h).

Its waves publish K/V tiles into LDS and bump a per-tile arrival counter;
a wave that needs tile t polls (bounded) until all NW waves have bumped it.
There is no workgroup barrier between the first and the final merge, so a
schedule in which some wave waits on a tile before every wave has produced
it would hang (the wait would run out and the wave compute on an unpublished
tile).  This test restates each wave's sequence of counter bumps, waits and
barriers and runs them under an event scheduler (always one runnable wave,
fixed or randomised choice).  It checks, for every shape the resident kernel
serves (S <= 256 at 32-row tiles, causal or not, probs or not, ring depth
L = 2 or 4, every launch rank): every wave finishes, and every tile is
published exactly NW times.

Restated from FaResident::run: tiles T = ceil(min(q0 + 256, Sq) + off) / 32)
(causal) or ceil(Sk / 32); wave tiles wtiles from tile_range; issue(0..L-1),
ahead(t < L) = publish t; step(t): publish t + L if t + L < T, then, when
t < wtiles, wait cnt[t] >= NW.  Waves 2j and 2j+1 of the SIMD ranking take
sub-blocks j and 7-j.
"""
import random

import pytest

BK = QW = 32
NQS = 8


def wtiles_of(q0, qw0, Sq, Sk, off, causal):
    kend = wkend = Sk
    if causal:
        kend = min(Sk, min(q0 + NQS * QW, Sq) + off)
        wkend = min(Sk, min(qw0 + QW, Sq) + off)
    ntiles = (kend + BK - 1) // BK
    wt = (wkend + BK - 1) // BK if qw0 < Sq else 0
    return ntiles, wt


def wave_programs(Sq, Sk, causal, probs, L, rank, n_qblk):
    nw = NQS
    off = Sk - Sq if causal else 0
    qb = n_qblk - 1 - rank if causal else rank
    q0 = qb * NQS * QW
    waves = []
    for rk in range(nw):
        simd = rk // 2
        sub = NQS - 1 - simd if rk & 1 else simd
        qw0 = q0 + sub * QW
        T, wt = wtiles_of(q0, qw0, Sq, Sk, off, causal)
        ops = [("barrier", 0)]  # the counters' clear is published by a barrier
        for t in range(min(L, T)):
            ops.append(("pub", t))
        for t in range(T):
            if t + L < T:
                ops.append(("pub", t + L))
            if t < wt:
                ops.append(("wait", t))
        waves.append(ops)
    return waves, nw


def run(waves, nw, rng=None):
    cnt = {}
    pos = [0] * len(waves)
    while True:
        at_barrier = {}
        runnable = []
        for w, ops in enumerate(waves):
            if pos[w] >= len(ops):
                continue
            kind, x = ops[pos[w]]
            if kind == "wait" and cnt.get(x, 0) < nw:
                continue
            if kind == "barrier":
                at_barrier.setdefault(x, []).append(w)
                continue
            runnable.append(w)
        # a barrier releases once every wave that has not finished stands at it
        live = [w for w in range(len(waves)) if pos[w] < len(waves[w])]
        for x, ws in at_barrier.items():
            if sorted(ws) == live:
                for w in ws:
                    pos[w] += 1
                runnable = None
                break
        if runnable is None:
            continue
        if not runnable:
            break
        w = rng.choice(runnable) if rng else runnable[0]
        kind, x = waves[w][pos[w]]
        if kind == "pub":
            cnt[x] = cnt.get(x, 0) + 1
        pos[w] += 1
    blocked = [w for w in range(len(waves)) if pos[w] < len(waves[w])]
    return blocked, cnt


@pytest.mark.parametrize("L", [2, 4])
@pytest.mark.parametrize("probs", [False, True])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("S", [1, 31, 32, 33, 64, 100, 200, 255, 256])
def test_every_tile_wait_ends(S, causal, probs, L):
    n_qblk = (S + NQS * QW - 1) // (NQS * QW)
    for rank in range(n_qblk):
        waves, nw = wave_programs(S, S, causal, probs, L, rank, n_qblk)
        T = max(sum(1 for k, _ in ops if k == "pub") for ops in waves)
        for rng in [None] + [random.Random(seed) for seed in range(10)]:
            blocked, cnt = run(waves, nw, rng)
            assert not blocked, f"waves {blocked} never finish"
            assert all(cnt.get(t, 0) == nw for t in range(T))  # every tile published by every wave


def test_a_missing_publication_is_caught():
    """The checker itself: drop one wave's publication of tile 1 and the
    schedule must block (a wave waits on tile 1 forever)."""
    waves, nw = wave_programs(256, 256, True, False, 4, 0, 1)
    victim = waves[3]
    waves[3] = [op for op in victim if op != ("pub", 1)]
    blocked, _ = run(waves, nw)
    assert blocked
