"""CPU checks of bench.py's contract with the round driver: the one-GPU
refusal, the algorithmic work it prices the roofline with, the buffer
rotation that keeps operands out of the Infinity Cache, and the CPU baseline
leg (the oracle, timed on the host)."""
import json
import math
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--no-cpu"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one MI355X" in r.stderr
    assert r.stdout.strip() == ""  # no JSON line for a configuration that was not measured


def test_headline_config_is_the_baseline_metric_shape():
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        metric = json.load(f)["metric"]
    assert metric == bench.METRIC
    B, H, Sq, Sk, D, causal, dtype, probs, kind = bench.CONFIGS["c1"]
    assert (B, H, Sq, Sk, D, causal, dtype, probs, kind) == (32, 8, 256, 256, 32, True, "f32", False, "fwd")
    assert "B32 H8 S256 D32" in metric


def test_forward_work_closed_form():
    # 4 * B * H * D flops per visible (query, key) pair; Q, K, V read once and O written once
    B, H, S, D = 32, 8, 256, 32
    flops, nbytes = bench.work(bench.CONFIGS["c1"])
    assert flops == 4.0 * B * H * D * (S * (S + 1) // 2)
    assert nbytes == 4 * B * H * S * D * 4
    # the drop-in: every pair visible, the [B][H][S][S] probs written
    flops, nbytes = bench.work(bench.CONFIGS["c1_legacy"])
    assert flops == 4.0 * B * H * D * S * S
    assert nbytes == 4 * B * H * S * D * 4 + 4 * B * H * S * S


def test_backward_and_decode_work_closed_form():
    B, H, S, D = 32, 8, 256, 32
    flops, nbytes = bench.work(bench.CONFIGS["c1_bwd_legacy"])
    assert flops == 8.0 * B * H * D * S * S  # dP, dV, dK, dQ
    assert nbytes == 4 * B * H * (S * S + 7 * S * D)  # P, Q, K, V, dO in; dQ, dK, dV out
    flops, nbytes = bench.work(bench.CONFIGS["c5"])
    B, H, kv, D = 64, 12, 2048, 64
    assert flops == 4.0 * B * H * D * kv
    assert nbytes == 4 * B * H * D * (1 + 2 * kv) + 4 * B * H * D  # q, K, V read; O written


def test_layer_work_is_its_three_calls():
    # QKV projection (T x E @ E x 3E), the drop-in attention (non-causal, probs
    # written), output projection (T x E @ E x E)
    B, H, S, D = 32, 8, 256, 32
    T, E = B * S, H * D
    flops, nbytes = bench.work(bench.CONFIGS["c1_layer"])
    assert flops == 2.0 * T * E * 3 * E + 4.0 * B * H * D * S * S + 2.0 * T * E * E
    assert nbytes == (4 * (T * E + E * 3 * E + 3 * E + T * 3 * E) + 4 * B * H * S * D * 4 + 4 * B * H * S * S
                      + 4 * (T * E + E * E + E + T * E))


@pytest.mark.parametrize("name", list(bench.CONFIGS))
def test_rotation_covers_the_infinity_cache(name):
    # the sets a config rotates over hold at least 1 GiB together (MI355X's
    # Infinity Cache is 256 MB), so a timed call's operands come from HBM
    cfg = bench.CONFIGS[name]
    sb = bench.set_bytes(cfg)
    assert sb > 0
    nsets = max(1, math.ceil(bench.ROTATE_BYTES / sb))
    assert nsets * sb >= bench.ROTATE_BYTES >= 4 * 256 * 10**6


def test_cpu_baseline_leg_times_the_oracle():
    info = bench.host_info()
    assert info["nproc"] >= 1 and info["affinity"] >= 1 and info["cpu_model"]
    r = bench.cpu_config("c1", 1, 0.05)  # at least one (b, h) pair, scaled to the whole problem
    assert r["threads"] == 1 and 1 <= r["pairs"] <= r["of_pairs"] == 256
    assert r["us_per_call"] > 0 and r["gflops"] > 0
