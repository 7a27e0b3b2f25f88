"""HipGPT's attention sub-layer through the drop-in C++ symbols, from C++.

tests/cpp/layer_dropin is a host program compiled with g++ against
include/hip_kernels.h and linked to libhipgpt_attn.so, as HipGPT's executables
would be (src/transformer_layer.cpp:214-222 forward, :285-286 backward).  It
runs QKV projection -> attention (probs) -> output projection -> attention
backward on the null stream and checks every stage against the oracle with
bar 1e-4 x max(1, max|want|).  The CPU test checks the program is built and
resolves every symbol; the GPU tests run it.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "layer_dropin")

# D = 32 (flash-path shape of the reference), 48 and 96 (padded), 128, 64 with
# S beyond a tile multiple; the last is c1's head shape on one sequence.
SHAPES = [(2, 64, 128, 4), (2, 100, 96, 2), (1, 70, 192, 2), (1, 33, 512, 4), (3, 45, 256, 4), (1, 256, 256, 8)]


def _run(*args, timeout=120):
    return subprocess.run([EXE, *map(str, args)], capture_output=True, text=True, timeout=timeout)


def test_program_built_and_linked():
    if not os.path.exists(EXE):
        pytest.skip("tests/cpp/layer_dropin not built (run __graft_entry__.build())")
    r = _run()  # usage error: exits before any HIP call
    assert r.returncode == 2 and "usage" in r.stderr
    r = _run(1, 8, 30, 4)  # E % H != 0 is refused by the program itself
    assert r.returncode == 2 and "bad shape" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("B,S,E,H", SHAPES)
def test_layer_dropin_matches_oracle(B, S, E, H):
    if not os.path.exists(EXE):
        pytest.fail("tests/cpp/layer_dropin not built")
    print(f"layer_dropin {B} {S} {E} {H}", flush=True)
    r = _run(B, S, E, H)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS" in r.stdout
