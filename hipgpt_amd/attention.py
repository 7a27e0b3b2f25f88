"""Host-side mirror of HipGPT's attention forward interface over libhipgpt_attn.so.

Tensors are torch device tensors (torch is only the allocator and stream
provider here); every call goes through the C ABI to the HIP kernels.

* :func:`launch_multihead_attention` -- HipGPT's launcher
  (``include/hip_kernels.h:39-43``, ``src/hip_kernels.cpp:404-451``): planar
  ``d_qkv = [Q|K|V]`` each ``[B*S, E]``, non-causal, probs written when given.
* :func:`qkv_planar` -- same layout, plus causal masking and a stream.
* :func:`launch_multihead_attention_backward` / :func:`attention_backward` --
  HipGPT's backward on the stored probs.
* :func:`fwd_lse_qkv_planar` / :func:`bwd_lse_qkv_planar` -- the training pair
  without a probs buffer: the forward keeps a per-row log-sum-exp and the
  backward recomputes P from it.
* :func:`attention` -- strided ``[B, S, H, D]`` views, fp32 or bf16 inputs.
* :func:`decode` -- one query row per sequence against ``kv_len`` keys,
  split-KV.
* :func:`decode_kvcache` -- one KV-cached generation step: append the new
  key/value row at each sequence's device-side length, attend, advance.
"""
from __future__ import annotations

import math

import torch

from . import _lib


def _ptr(t):
    return 0 if t is None else t.data_ptr()


def _stream(stream):
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _need_cuda(name, t, dtype=None):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a CUDA (HIP) tensor")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")


def launch_multihead_attention(d_qkv, d_output, d_attn_probs, B, S, E, H):
    """HipGPT ``launch_multihead_attention`` (drop-in semantics).

    The C++ symbol aborts the process on ``H <= 0 or E % H != 0``
    (``src/hip_kernels.cpp:410-413``); this Python mirror raises the same
    message as ``ValueError`` before reaching it.  Launches on the null
    stream, like the reference.
    """
    if H <= 0 or E % H != 0:
        raise ValueError(f"Bad MHA config: E={E} H={H}")
    _need_cuda("d_qkv", d_qkv, torch.float32)
    _need_cuda("d_output", d_output, torch.float32)
    n = B * S * E
    if d_qkv.numel() < 3 * n or d_output.numel() < n:
        raise ValueError("d_qkv / d_output too small for B*S*E")
    if d_attn_probs is not None:
        _need_cuda("d_attn_probs", d_attn_probs, torch.float32)
        if d_attn_probs.numel() < B * H * S * S:
            raise ValueError("d_attn_probs too small for B*H*S*S")
    for t in (d_qkv, d_output, d_attn_probs):
        if t is not None and not t.is_contiguous():
            raise ValueError("launch_multihead_attention needs contiguous buffers")
    _lib.lib().hipgpt_launch_multihead_attention(
        _ptr(d_qkv), _ptr(d_output), _ptr(d_attn_probs), B, S, E, H
    )


def _need_numel(name, t, n):
    _need_cuda(name, t, torch.float32)
    if t.numel() < n or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 tensor with >= {n} elements")


def launch_scaled_dot_product(Q, K, scores, B, S, D):
    """HipGPT ``launch_scaled_dot_product`` (src/hip_kernels.cpp:455-472):
    scores[b*S+i, j] = Q[b*S+i] . K[b*S+j] / sqrt(D); null stream."""
    _need_numel("Q", Q, B * S * D)
    _need_numel("K", K, B * S * D)
    _need_numel("scores", scores, B * S * S)
    _lib.lib().hipgpt_launch_scaled_dot_product(_ptr(Q), _ptr(K), _ptr(scores), B, S, D)


def launch_softmax(scores, softmax_out, B, S):
    """HipGPT ``launch_softmax`` (src/hip_kernels.cpp:478-509): row softmax
    of [B*S, S]; null stream."""
    _need_numel("scores", scores, B * S * S)
    _need_numel("softmax_out", softmax_out, B * S * S)
    _lib.lib().hipgpt_launch_softmax(_ptr(scores), _ptr(softmax_out), B, S)


def launch_attention_weighted_sum(softmax, V, output, B, S, D):
    """HipGPT ``launch_attention_weighted_sum`` (src/hip_kernels.cpp:512-532):
    output[b*S+i] = sum_j softmax[b*S+i, j] V[b*S+j]; null stream."""
    _need_numel("softmax", softmax, B * S * S)
    _need_numel("V", V, B * S * D)
    _need_numel("output", output, B * S * D)
    _lib.lib().hipgpt_launch_attention_weighted_sum(_ptr(softmax), _ptr(V), _ptr(output), B, S, D)


def launch_multihead_attention_backward(d_grad_attn_output, d_qkv, d_softmax, d_grad_qkv, B, S, E, H):
    """HipGPT ``launch_multihead_attention_backward`` (src/hip_kernels.cpp:1245-1272):
    planar [dQ|dK|dV] from dO, the forward's planar Q|K|V and its probs.
    Null stream; the C++ symbol aborts on a bad head split (raised here)."""
    if H <= 0 or E % H != 0:
        raise ValueError(f"Bad MHA config: E={E} H={H}")
    n = B * S * E
    _need_numel("d_grad_attn_output", d_grad_attn_output, n)
    _need_numel("d_qkv", d_qkv, 3 * n)
    _need_numel("d_softmax", d_softmax, B * H * S * S)
    _need_numel("d_grad_qkv", d_grad_qkv, 3 * n)
    _lib.lib().hipgpt_launch_multihead_attention_backward(
        _ptr(d_grad_attn_output), _ptr(d_qkv), _ptr(d_softmax), _ptr(d_grad_qkv), B, S, E, H)


def attention_backward(grad_out, qkv, probs, grad_qkv, B, S, E, H, causal=False, workspace=None, stream=None):
    """Backward with a caller workspace and stream; ``causal`` skips the
    probs tiles a causal forward zeroed."""
    n = B * S * E
    _need_numel("grad_out", grad_out, n)
    _need_numel("qkv", qkv, 3 * n)
    _need_numel("probs", probs, B * H * S * S)
    _need_numel("grad_qkv", grad_qkv, 3 * n)
    need = int(_lib.lib().hipgpt_attn_bwd_workspace_bytes(B, S, H))
    if workspace is None:
        workspace = torch.empty(max(1, need // 4), device=qkv.device, dtype=torch.float32)
    rc = _lib.lib().hipgpt_attn_bwd_qkv_planar(
        _ptr(grad_out), _ptr(qkv), _ptr(probs), _ptr(grad_qkv), B, S, E, H, int(bool(causal)),
        _ptr(workspace), workspace.numel() * workspace.element_size(), _stream(stream))
    _lib.check(rc, "hipgpt_attn_bwd_qkv_planar")
    return grad_qkv


def qkv_planar(d_qkv, d_output, d_attn_probs, B, S, E, H, causal=False, stream=None):
    """Planar-layout forward with causal masking and an explicit stream."""
    _need_cuda("d_qkv", d_qkv, torch.float32)
    _need_cuda("d_output", d_output, torch.float32)
    if d_qkv.numel() < 3 * B * S * E or d_output.numel() < B * S * E:
        raise ValueError("d_qkv / d_output too small for B*S*E")
    if d_attn_probs is not None:
        _need_cuda("d_attn_probs", d_attn_probs, torch.float32)
        if d_attn_probs.numel() < B * H * S * S:
            raise ValueError("d_attn_probs too small for B*H*S*S")
    rc = _lib.lib().hipgpt_attn_qkv_planar(
        _ptr(d_qkv), _ptr(d_output), _ptr(d_attn_probs), B, S, E, H, int(bool(causal)),
        _stream(stream),
    )
    _lib.check(rc, "hipgpt_attn_qkv_planar")


def fwd_lse_qkv_planar(d_qkv, d_output, lse, B, S, E, H, causal=False, stream=None):
    """Training forward without probs: O and the row log-sum-exp
    ``lse`` [B, H, S] (natural log of the softmax denominator of q.k/sqrt(D))."""
    _need_cuda("d_qkv", d_qkv, torch.float32)
    _need_cuda("d_output", d_output, torch.float32)
    _need_cuda("lse", lse, torch.float32)
    _need_numel("d_qkv", d_qkv, 3 * B * S * E)
    _need_numel("d_output", d_output, B * S * E)
    _need_numel("lse", lse, B * H * S)
    rc = _lib.lib().hipgpt_attn_fwd_lse_qkv_planar(
        _ptr(d_qkv), _ptr(d_output), _ptr(lse), B, S, E, H, int(bool(causal)), _stream(stream))
    _lib.check(rc, "hipgpt_attn_fwd_lse_qkv_planar")


def bwd_lse_qkv_planar(grad_out, qkv, out, lse, grad_qkv, B, S, E, H, causal=False, workspace=None, stream=None):
    """Backward of :func:`fwd_lse_qkv_planar` from its ``out`` and ``lse``
    (P recomputed per tile; no probs buffer)."""
    n = B * S * E
    for name, t, k in (("grad_out", grad_out, n), ("qkv", qkv, 3 * n), ("out", out, n), ("lse", lse, B * H * S),
                       ("grad_qkv", grad_qkv, 3 * n)):
        _need_cuda(name, t, torch.float32)
        _need_numel(name, t, k)
    # head dims other than 32 / 64 pass the row dots dO . O between their two
    # kernels through a B*H*S workspace
    if workspace is None and E // H not in (32, 64):
        need = int(_lib.lib().hipgpt_attn_bwd_workspace_bytes(B, S, H))
        workspace = torch.empty(max(1, need // 4), device=qkv.device, dtype=torch.float32)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = _lib.lib().hipgpt_attn_bwd_lse_qkv_planar(
        _ptr(grad_out), _ptr(qkv), _ptr(out), _ptr(lse), _ptr(grad_qkv), B, S, E, H, int(bool(causal)),
        _ptr(workspace), ws_bytes, _stream(stream))
    _lib.check(rc, "hipgpt_attn_bwd_lse_qkv_planar")
    return grad_qkv


def _bshd_strides(t, name):
    if t.dim() != 4:
        raise ValueError(f"{name} must be [B, S, H, D]")
    if t.stride(3) != 1:
        raise ValueError(f"{name} must be contiguous in D")
    return t.stride(0), t.stride(1), t.stride(2)


def attention(q, k, v, out=None, probs=None, causal=False, scale=None, stream=None):
    """softmax(q k^T * scale) v over ``[B, S, H, D]`` views; returns fp32 ``out``.

    q: [B, Sq, H, D], k/v: [B, Sk, H, D], all float32 or all bfloat16 (bf16
    runs bf16 MFMA with fp32 accumulation).  ``probs`` (optional) is fp32
    ``[B, H, Sq, Sk]``.  ``causal`` masks keys j > i + (Sk - Sq).
    """
    for name, t in (("q", q), ("k", k), ("v", v)):
        _need_cuda(name, t)
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("q, k, v must all be float32 or all bfloat16")
    B, Sq, H, D = q.shape
    if k.shape[0] != B or k.shape[2] != H or k.shape[3] != D or v.shape != k.shape:
        raise ValueError("k, v must be [B, Sk, H, D] matching q")
    Sk = k.shape[1]
    if out is None:
        out = torch.empty((B, Sq, H, D), device=q.device, dtype=torch.float32)
    _need_cuda("out", out, torch.float32)
    if tuple(out.shape) != (B, Sq, H, D):
        raise ValueError("out must be [B, Sq, H, D]")
    if probs is not None:
        _need_cuda("probs", probs, torch.float32)
        if tuple(probs.shape) != (B, H, Sq, Sk) or not probs.is_contiguous():
            raise ValueError("probs must be contiguous [B, H, Sq, Sk]")
    qs, ks, vs, os_ = (_bshd_strides(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v"), (out, "out")))
    dtype = _lib.F32 if q.dtype == torch.float32 else _lib.BF16
    sc = -1.0 if scale is None else float(scale)
    rc = _lib.lib().hipgpt_attn_fwd(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(probs), B, H, Sq, Sk, D,
        *qs, *ks, *vs, *os_, sc, int(bool(causal)), dtype, _stream(stream),
    )
    _lib.check(rc, "hipgpt_attn_fwd")
    return out


def decode_workspace_bytes(B, H, D, num_splits):
    return int(_lib.lib().hipgpt_attn_decode_workspace_bytes(B, H, D, num_splits))


def decode_default_splits(B, H, kv_len):
    return int(_lib.lib().hipgpt_attn_decode_default_splits(B, H, kv_len))


def decode(q, k, v, out=None, num_splits=None, workspace=None, scale=None, stream=None):
    """One decode step: q [B, 1, H, D] against k/v [B, kv_len, H, D] (fp32).

    Split-KV with ``num_splits`` partitions (default: the library's choice);
    ``workspace`` is a caller-owned device buffer (allocated here if None).
    """
    for name, t in (("q", q), ("k", k), ("v", v)):
        _need_cuda(name, t, torch.float32)
    B, one, H, D = q.shape
    if one != 1:
        raise ValueError("q must be [B, 1, H, D]")
    kv = k.shape[1]
    if tuple(k.shape) != (B, kv, H, D) or v.shape != k.shape:
        raise ValueError("k, v must be [B, kv_len, H, D]")
    if out is None:
        out = torch.empty((B, 1, H, D), device=q.device, dtype=torch.float32)
    _need_cuda("out", out, torch.float32)
    ns = decode_default_splits(B, H, kv) if num_splits is None else int(num_splits)
    ns = max(1, min(ns, kv))
    need = decode_workspace_bytes(B, H, D, ns)
    if workspace is None and need > 0:
        workspace = torch.empty(need // 4, device=q.device, dtype=torch.float32)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    qs, ks, vs, os_ = (_bshd_strides(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v"), (out, "out")))
    sc = -1.0 if scale is None else float(scale)
    rc = _lib.lib().hipgpt_attn_decode(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, H, kv, D,
        qs[0], qs[2], *ks, *vs, os_[0], os_[2],
        sc, ns, _ptr(workspace), ws_bytes, _stream(stream),
    )
    _lib.check(rc, "hipgpt_attn_decode")
    return out


def _bhd_strides(t, name, B, H, D):
    if tuple(t.shape) != (B, H, D) or t.stride(2) != 1:
        raise ValueError(f"{name} must be [B, H, D] with contiguous D")
    return t.stride(0), t.stride(1)


def decode_kvcache(q, k_new, v_new, k_cache, v_cache, lens, out=None, advance=True, num_splits=None,
                   workspace=None, scale=None, stream=None):
    """One KV-cached decode step over sequences of different lengths.

    q, k_new, v_new: [B, H, D] fp32 (the step's projections); k_cache,
    v_cache: [B, max_len, H, D] fp32 with the same strides; lens: int32
    device tensor [B] of cached rows.  Writes k_new / v_new at row lens[b],
    attends q over the lens[b] + 1 rows and (``advance``) increments lens on
    the device.  Sequences at capacity get NaN and are left unchanged.
    """
    for name, t in (("q", q), ("k_new", k_new), ("v_new", v_new), ("k_cache", k_cache), ("v_cache", v_cache)):
        _need_cuda(name, t, torch.float32)
    _need_cuda("lens", lens, torch.int32)
    B, H, D = q.shape
    if k_cache.dim() != 4 or k_cache.shape[0] != B or k_cache.shape[2] != H or k_cache.shape[3] != D:
        raise ValueError("k_cache must be [B, max_len, H, D]")
    if v_cache.shape != k_cache.shape or v_cache.stride() != k_cache.stride() or k_cache.stride(3) != 1:
        raise ValueError("v_cache must match k_cache in shape and strides, D contiguous")
    if lens.numel() != B or not lens.is_contiguous():
        raise ValueError("lens must be a contiguous int32 tensor of B elements")
    max_len = k_cache.shape[1]
    if out is None:
        out = torch.empty((B, H, D), device=q.device, dtype=torch.float32)
    _need_cuda("out", out, torch.float32)
    qs = _bhd_strides(q, "q", B, H, D)
    ks = _bhd_strides(k_new, "k_new", B, H, D)
    vs = _bhd_strides(v_new, "v_new", B, H, D)
    os_ = _bhd_strides(out, "out", B, H, D)
    ns = decode_default_splits(B, H, max_len) if num_splits is None else int(num_splits)
    ns = max(1, min(ns, max_len))
    need = decode_workspace_bytes(B, H, D, ns)
    if workspace is None and need > 0:
        workspace = torch.empty(need // 4, device=q.device, dtype=torch.float32)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    sc = -1.0 if scale is None else float(scale)
    rc = _lib.lib().hipgpt_attn_decode_kvcache(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache), _ptr(lens), _ptr(out),
        B, H, D, max_len, *qs, *ks, *vs, k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), *os_,
        sc, ns, int(bool(advance)), _ptr(workspace), ws_bytes, _stream(stream))
    _lib.check(rc, "hipgpt_attn_decode_kvcache")
    return out


def default_scale(D):
    return 1.0 / math.sqrt(D)
