"""CPU tests pinning the oracle's restatement of HipGPT's projection GEMMs
(launch_matmul / launch_matmul_add_bias, src/hip_kernels.cpp:70-154).

What fixes the restatement independently of its own formula:
  * integer-valued inputs, where every partial sum is exact in fp32, so the
    result must equal numpy's int64 product (a transposed operand, a wrong
    index or a dropped term changes the integers);
  * random inputs against a float64 product within the dot-product rounding
    bound gamma_N * sum|a||b| (Higham, Accuracy and Stability, 3.1);
  * bias added once per output column, after the sum; empty grids.
Bit-exactness against the reference's own HIP kernel is checked on the GPU
(tests/test_gemm_gpu.py).
"""
import numpy as np
import pytest

import oracle as O

U32 = 2.0 ** -24


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (33, 64, 17), (64, 256, 96), (7, 300, 5)])
def test_integer_inputs_exact(M, N, K):
    rng = np.random.default_rng(M * 1000 + N * 10 + K)
    A = rng.integers(-8, 9, size=(M, N)).astype(np.float32)
    B = rng.integers(-8, 9, size=(N, K)).astype(np.float32)
    bias = rng.integers(-100, 101, size=K).astype(np.float32)
    want = A.astype(np.int64) @ B.astype(np.int64) + bias.astype(np.int64)
    got = O.matmul_add_bias(A, B, bias, M, N, K)
    assert np.array_equal(got.astype(np.int64), want)
    got0 = O.matmul_add_bias(A, B, None, M, N, K)
    assert np.array_equal(got0.astype(np.int64), A.astype(np.int64) @ B.astype(np.int64))


@pytest.mark.parametrize("M,N,K", [(16, 256, 48), (9, 1024, 13), (40, 33, 40)])
def test_random_inputs_within_rounding_bound(M, N, K):
    x = O.fill_normal(0x6E4D + N, M * N + N * K + K)
    A = x[: M * N].reshape(M, N)
    B = x[M * N: M * N + N * K].reshape(N, K)
    bias = x[M * N + N * K:]
    got = O.matmul_add_bias(A, B, bias, M, N, K).astype(np.float64)
    exact = A.astype(np.float64) @ B.astype(np.float64) + bias
    gamma = N * U32 / (1 - N * U32)
    bound = gamma * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)) + U32 * np.abs(exact) + 1e-30
    assert (np.abs(got - exact) <= bound).all()
    # and it is a real fp32 result, not a double one rounded once
    assert np.abs(got - exact).max() > 0


def test_empty_and_degenerate_shapes():
    A = np.ones((2, 3), np.float32)
    B = np.ones((3, 4), np.float32)
    bias = np.arange(4, dtype=np.float32)
    # N = 0: the reference's tile loop does not run, C = bias
    got = O.matmul_add_bias(np.zeros((2, 0), np.float32), np.zeros((0, 4), np.float32), bias, 2, 0, 4)
    assert np.array_equal(got, np.tile(bias, (2, 1)))
    assert np.array_equal(O.matmul_add_bias(A, B, bias, 2, 3, 4), 3 + np.tile(bias, (2, 1)))
