"""GPU parity of the projection GEMMs (launch_matmul_add_bias / launch_matmul,
src/hip_kernels.cpp:70-154) against the oracle restatement, and of the
oracle against the reference's own HIP kernels (oracle/_ref).

Bars (fp32): the MFMA GEMM sums in a different order from the reference's
sequential loop, so it is held to the same accuracy as the reference's own
arithmetic: its max error against a float64 product is at most twice the
oracle's (and never above the dot-product bound gamma_N * sum|a||b|).  bf16
outputs are the fp32 result rounded to nearest even: within half a bf16 ulp
of the oracle (plus the fp32 bar).
"""
import numpy as np
import pytest
import torch

import oracle as O
from hipgpt_amd import projection as P

pytestmark = pytest.mark.gpu

U32 = 2.0 ** -24


def dev_t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().float().cpu().numpy()


def operands(seed, M, N, K):
    x = O.fill_normal(seed, M * N + N * K + K)
    return x[: M * N].reshape(M, N), x[M * N: M * N + N * K].reshape(N, K), x[M * N + N * K:].copy()


def check_fp32(got, A, B, bias, want):
    """got, want: [M, K]; want is the oracle's result on the same operands."""
    exact = A.astype(np.float64) @ B.astype(np.float64)
    if bias is not None:
        exact = exact + bias
    N = A.shape[1]
    gamma = N * U32 / (1 - N * U32)
    bound = gamma * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)) + 2 * U32 * np.abs(exact) + 1e-30
    err = np.abs(got.astype(np.float64) - exact)
    assert (err <= bound).all(), float((err / bound).max())
    ref_err = np.abs(want.astype(np.float64) - exact).max()
    assert err.max() <= max(2 * ref_err, 4 * U32 * np.abs(exact).max()), (err.max(), ref_err)


# (M, N, K) in the reference's naming: A [M, N], B [N, K], C [M, K].
# Vector path (N, K multiples of 4), ragged edges of both tile shapes, the
# scalar path (N or K not a multiple of 4), and a tiny problem.  An inner dim
# N that is a multiple of 32 takes the whole-k-tile loads; (70, 64, 100) and
# (129, 96, 260) give them a partial column tile and partial row tiles.
SHAPES = [(1, 4, 4), (3, 5, 7), (64, 256, 256), (130, 256, 768), (97, 36, 52), (200, 1024, 256),
          (33, 33, 33), (640, 256, 12), (5, 2, 1000), (70, 64, 100), (129, 96, 260)]


@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_drop_in_matmul_matches_oracle(dev, M, N, K, with_bias):
    A, B, bias = operands(M * 131 + N * 7 + K, M, N, K)
    want = O.matmul_add_bias(A, B, bias if with_bias else None, M, N, K)
    dA, dB, db = dev_t(A), dev_t(B), dev_t(bias)
    dC = torch.full((M, K), float("nan"), device=dev)
    if with_bias:
        P.launch_matmul_add_bias(dA, dB, db, dC, M, N, K)
    else:
        P.launch_matmul(dA, dB, dC, M, N, K)
    check_fp32(host(dC), A, B, bias if with_bias else None, want)


@pytest.mark.parametrize("M,N,K", [(3, 5, 7), (64, 256, 256), (97, 36, 52), (130, 256, 768)])
def test_oracle_bit_exact_with_reference_kernel(dev, M, N, K):
    if not O.ref_available():
        pytest.skip("reference build oracle/_ref missing")
    ref = O.ref_lib()
    A, B, bias = operands(M + N + K, M, N, K)
    dA, dB, db = dev_t(A), dev_t(B), dev_t(bias)
    dC = torch.full((M, K), float("nan"), device=dev)
    ref.matmul_add_bias(dA.data_ptr(), dB.data_ptr(), db.data_ptr(), dC.data_ptr(), M, N, K)
    assert np.array_equal(host(dC), O.matmul_add_bias(A, B, bias, M, N, K))
    ref.matmul(dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), M, N, K)
    assert np.array_equal(host(dC), O.matmul_add_bias(A, B, None, M, N, K))


def test_inner_dim_zero_gives_bias(dev):
    bias = dev_t(np.arange(8, dtype=np.float32))
    C = torch.full((3, 8), float("nan"), device=dev)
    empty = torch.zeros(1, device=dev)
    P.launch_matmul_add_bias(empty, empty, bias, C, 3, 0, 8)
    assert np.array_equal(host(C), np.tile(np.arange(8, dtype=np.float32), (3, 1)))


@pytest.mark.parametrize("planar", [False, True])
@pytest.mark.parametrize("T,E", [(96, 64), (256, 256), (75, 96)])
def test_qkv_projection_layouts(dev, T, E, planar):
    x, w, b = operands(T * 3 + E, T, E, 3 * E)
    want = O.matmul_add_bias(x, w, b, T, E, 3 * E)
    got = host(P.qkv_projection(dev_t(x), dev_t(w), dev_t(b), planar=planar))
    if planar:
        assert got.shape == (3, T, E)
        got = np.concatenate([got[0], got[1], got[2]], axis=1)  # back to [T, 3E] rows
    check_fp32(got, x, w, b, want)


@pytest.mark.parametrize("M,N,K", [(130, 256, 768), (64, 96, 40)])
def test_bf16_output_is_rounded_fp32(dev, M, N, K):
    A, B, bias = operands(7 * M + K, M, N, K)
    want = O.matmul_add_bias(A, B, bias, M, N, K)
    got = host(P.gemm_bias(dev_t(A), dev_t(B), dev_t(bias), out_dtype=torch.bfloat16))
    # half a bf16 ulp (2^-8 relative) of rounding, plus the fp32 difference
    tol = np.abs(want) * 2.0 ** -8 + 1e-4
    assert (np.abs(got - want) <= tol).all()


def test_strided_operands_and_column_planes(dev):
    # A and W as column windows of wider buffers; output split in 4 planes
    M, K, N = 70, 48, 64
    big_a = torch.randn(M, 80, device=dev)
    big_w = torch.randn(K, 100, device=dev)
    A, W = big_a[:, 8:8 + K], big_w[:, 20:20 + N]
    bias = torch.randn(N, device=dev)
    out = torch.full((4 * M * 16,), float("nan"), device=dev)
    P.gemm_bias(A, W, bias, out=out, seg_w=16, seg_stride=M * 16)
    got = host(out).reshape(4, M, 16)
    got = np.concatenate(list(got), axis=1)
    An, Wn, bn = host(A), host(W), host(bias)
    want = O.matmul_add_bias(An, Wn, bn, M, K, N)
    check_fp32(got, An, Wn, bn, want)


def test_baseline_layer_shapes_every_row(dev):
    """The c1 layer's projections (T = 32*256 tokens, E = 256): QKV
    [8192, 256] x [256, 768] and out-projection [8192, 256] x [256, 256],
    every output element checked (the scalar C oracle takes ~1 s here)."""
    T, E = 8192, 256
    for N_out in (3 * E, E):
        A, B, bias = operands(0x51 + N_out, T, E, N_out)
        got = host(P.gemm_bias(dev_t(A), dev_t(B), dev_t(bias)))
        want = O.matmul_add_bias(A, B, bias, T, E, N_out)
        check_fp32(got, A, B, bias, want)
