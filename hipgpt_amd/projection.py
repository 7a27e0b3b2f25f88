"""Host-side mirror of HipGPT's projection GEMMs over libhipgpt_attn.so.

The QKV projection and the output projection around the attention
(``src/transformer_layer.cpp:217``, ``:220``) are ``launch_matmul_add_bias``
calls (``include/hip_kernels.h:7``, ``src/hip_kernels.cpp:113-154``).  Every
call goes through the C ABI to the fp32 MFMA GEMM; torch only provides
device memory and streams.

* :func:`launch_matmul_add_bias`, :func:`launch_matmul` -- the reference's
  signatures and naming: ``A [M, N] @ B [N, K] (+ bias [K]) -> C [M, K]``,
  null stream.
* :func:`gemm_bias` -- strided ``A [M, K] @ W [K, N] + bias`` with an explicit
  stream, fp32 or bf16 output, and an optional split of the output columns
  into planes.
* :func:`qkv_projection` -- ``x [T, E] @ w_qkv [E, 3E] + b_qkv`` written as the
  reference's ``[T, 3E]`` rows or as the planar ``[3, T, E]`` buffer the
  attention launchers read.
"""
from __future__ import annotations

import torch

from . import _lib
from .attention import _need_cuda, _need_numel, _ptr, _stream


def launch_matmul_add_bias(A, B, bias, C, M, N, K):
    """HipGPT ``launch_matmul_add_bias``: ``C[M, K] = A[M, N] @ B[N, K] + bias[K]``."""
    if M <= 0 or K <= 0:
        return
    n = max(N, 0)
    _need_numel("A", A, M * n)
    _need_numel("B", B, n * K)
    _need_numel("bias", bias, K)
    _need_numel("C", C, M * K)
    _lib.lib().hipgpt_launch_matmul_add_bias(_ptr(A), _ptr(B), _ptr(bias), _ptr(C), M, N, K)


def launch_matmul(A, B, C, M, N, K):
    """HipGPT ``launch_matmul``: ``C[M, K] = A[M, N] @ B[N, K]``."""
    if M <= 0 or K <= 0:
        return
    n = max(N, 0)
    _need_numel("A", A, M * n)
    _need_numel("B", B, n * K)
    _need_numel("C", C, M * K)
    _lib.lib().hipgpt_launch_matmul(_ptr(A), _ptr(B), _ptr(C), M, N, K)


def gemm_bias(A, W, bias=None, out=None, out_dtype=torch.float32, seg_w=None, seg_stride=0, ldc=None,
              stream=None):
    """``A [M, K] @ W [K, N] (+ bias [N])`` on fp32 MFMA.

    A and W are 2-D float32 tensors with unit column stride (any row stride).
    Output column ``n`` is stored at ``out + (n // seg_w) * seg_stride + m * ldc
    + n % seg_w`` (elements); the defaults give a contiguous ``[M, N]`` result.
    """
    _need_cuda("A", A, torch.float32)
    _need_cuda("W", W, torch.float32)
    if A.dim() != 2 or W.dim() != 2 or A.shape[1] != W.shape[0]:
        raise ValueError("A must be [M, K] and W [K, N]")
    if (A.shape[1] > 1 and A.stride(1) != 1) or (W.shape[1] > 1 and W.stride(1) != 1):
        raise ValueError("A and W need unit column stride")
    M, K = A.shape
    N = W.shape[1]
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("out_dtype must be float32 or bfloat16")
    if bias is not None:
        _need_numel("bias", bias, N)
    if seg_w is None:
        seg_w = N
    if ldc is None:
        ldc = seg_w
    if out is None:
        if seg_w != N:
            raise ValueError("pass `out` when splitting the output columns")
        out = torch.empty((M, N), device=A.device, dtype=out_dtype)
    _need_cuda("out", out, out_dtype)
    need = (N - 1) // seg_w * seg_stride + (M - 1) * ldc + min(seg_w, N)
    if out.numel() < need or not out.is_contiguous():
        raise ValueError(f"out must be contiguous with >= {need} elements")
    dt = _lib.F32 if out_dtype == torch.float32 else _lib.BF16
    rc = _lib.lib().hipgpt_gemm_bias(
        _ptr(A), _ptr(W), _ptr(bias), _ptr(out), M, N, K, A.stride(0), W.stride(0), ldc, seg_w, seg_stride,
        dt, _stream(stream))
    _lib.check(rc, "hipgpt_gemm_bias")
    return out


def qkv_projection(x, w_qkv, b_qkv, out=None, planar=False, out_dtype=torch.float32, stream=None):
    """HipGPT's QKV projection ``x [T, E] @ w_qkv [E, 3E] + b_qkv [3E]``.

    ``planar=False`` returns the reference's ``[T, 3E]`` rows;
    ``planar=True`` returns ``[3, T, E]`` (plane p, row t = projection p of
    token t), the layout ``launch_multihead_attention`` reads.
    """
    _need_cuda("x", x, torch.float32)
    T, E = x.shape
    _need_numel("x", x, T * E)
    _need_numel("w_qkv", w_qkv, E * 3 * E)
    _need_numel("b_qkv", b_qkv, 3 * E)
    shape = (3, T, E) if planar else (T, 3 * E)
    if out is None:
        out = torch.empty(shape, device=x.device, dtype=out_dtype)
    _need_cuda("out", out, out_dtype)
    if out.numel() < 3 * T * E or not out.is_contiguous():
        raise ValueError("out must be contiguous with 3*T*E elements")
    dt = _lib.F32 if out_dtype == torch.float32 else _lib.BF16
    layout = _lib.QKV_PLANAR if planar else _lib.QKV_ROWS
    rc = _lib.lib().hipgpt_qkv_projection(_ptr(x), _ptr(w_qkv), _ptr(b_qkv), _ptr(out), T, E, layout, dt,
                                          _stream(stream))
    _lib.check(rc, "hipgpt_qkv_projection")
    return out
