"""ctypes binding of oracle/liboracle_attn.so (attn_oracle.h) and of the
reference build oracle/_ref/libref_hip_kernels.so.

TEST INFRASTRUCTURE ONLY (the checker / CPU baseline; never the product).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle_attn.so")
REF_SO = os.path.join(HERE, "_ref", "libref_hip_kernels.so")

FLASH = 0
FALLBACK = 1

__all__ = [
    "ORACLE_SO", "REF_SO", "FLASH", "FALLBACK", "splitmix64", "fill_normal",
    "round_bf16", "attention", "launch_multihead_attention", "ref_available",
    "ref_lib", "planar_qkv", "seeded_planar", "seeded_bshd", "scaled_dot_product",
    "softmax_rows", "attention_weighted_sum", "mha_backward", "matmul_add_bias",
]


class _Problem(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("probs", ctypes.c_void_p),
        ("B", ctypes.c_int), ("H", ctypes.c_int), ("Sq", ctypes.c_int),
        ("Sk", ctypes.c_int), ("D", ctypes.c_int),
        ("q_bs", ctypes.c_int64), ("q_ts", ctypes.c_int64), ("q_hs", ctypes.c_int64),
        ("k_bs", ctypes.c_int64), ("k_ts", ctypes.c_int64), ("k_hs", ctypes.c_int64),
        ("v_bs", ctypes.c_int64), ("v_ts", ctypes.c_int64), ("v_hs", ctypes.c_int64),
        ("o_bs", ctypes.c_int64), ("o_ts", ctypes.c_int64), ("o_hs", ctypes.c_int64),
        ("causal", ctypes.c_int), ("variant", ctypes.c_int),
    ]


_lib = None


def _oracle():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle`")
        L = ctypes.CDLL(ORACLE_SO)
        L.oracle_splitmix64.restype = ctypes.c_uint64
        L.oracle_splitmix64.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.oracle_fill_normal.restype = None
        L.oracle_fill_normal.argtypes = [ctypes.c_uint64, ctypes.c_void_p, ctypes.c_size_t]
        L.oracle_round_bf16.restype = None
        L.oracle_round_bf16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        for fn in ("oracle_attention", "oracle_attention_f64"):
            getattr(L, fn).restype = ctypes.c_int
            getattr(L, fn).argtypes = [ctypes.POINTER(_Problem), ctypes.c_int]
        L.oracle_attention_pairs.restype = ctypes.c_int
        L.oracle_attention_pairs.argtypes = [ctypes.POINTER(_Problem), ctypes.c_void_p,
                                             ctypes.c_int, ctypes.c_int]
        for fn in ("oracle_scaled_dot_product", "oracle_attention_weighted_sum"):
            getattr(L, fn).restype = None
            getattr(L, fn).argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 4
        L.oracle_softmax_rows.restype = None
        L.oracle_softmax_rows.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int] * 3
        L.oracle_mha_backward.restype = ctypes.c_int
        L.oracle_mha_backward.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 4
        L.oracle_mha_backward_mt.restype = ctypes.c_int
        L.oracle_mha_backward_mt.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 5
        L.oracle_matmul_add_bias.restype = ctypes.c_int
        L.oracle_matmul_add_bias.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 3
        L.oracle_launch_multihead_attention.restype = ctypes.c_int
        L.oracle_launch_multihead_attention.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ]
        _lib = L
    return _lib


def splitmix64(seed: int, n: int):
    st = ctypes.c_uint64(seed)
    return [_oracle().oracle_splitmix64(ctypes.byref(st)) for _ in range(n)]


def fill_normal(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _oracle().oracle_fill_normal(seed, out.ctypes.data, n)
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    _oracle().oracle_round_bf16(x.ctypes.data, out.ctypes.data, x.size)
    return out


def _el_strides(a):
    return tuple(s // a.itemsize for s in a.strides)


def attention(q, k, v, causal=False, variant=FALLBACK, want_probs=False, f64=False,
              nthreads=None, pairs=None):
    """Oracle over [B, S, H, D] float32 numpy views (any strides, D contiguous).

    variant FLASH / FALLBACK selects the restatement of
    flash_attention_kernel (src/hip_kernels.cpp:263-325) or the fallback
    (:329-402); f64 selects the textbook double-precision form.
    Returns (out [B, Sq, H, D], probs [B, H, Sq, Sk] or None).
    """
    for a in (q, k, v):
        if a.dtype != np.float32 or a.ndim != 4 or a.strides[3] != 4:
            raise ValueError("oracle inputs must be float32 [B,S,H,D] with contiguous D")
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    out = np.zeros((B, Sq, H, D), dtype=np.float32)
    probs = np.zeros((B, H, Sq, Sk), dtype=np.float32) if want_probs else None
    p = _Problem()
    p.q, p.k, p.v = q.ctypes.data, k.ctypes.data, v.ctypes.data
    p.o = out.ctypes.data
    p.probs = probs.ctypes.data if probs is not None else None
    p.B, p.H, p.Sq, p.Sk, p.D = B, H, Sq, Sk, D
    (p.q_bs, p.q_ts, p.q_hs, _) = _el_strides(q)
    (p.k_bs, p.k_ts, p.k_hs, _) = _el_strides(k)
    (p.v_bs, p.v_ts, p.v_hs, _) = _el_strides(v)
    (p.o_bs, p.o_ts, p.o_hs, _) = _el_strides(out)
    p.causal = int(bool(causal))
    p.variant = variant
    nt = nthreads if nthreads is not None else min(8, os.cpu_count() or 1)
    L = _oracle()
    if pairs is not None:
        pr = np.ascontiguousarray(np.asarray(pairs, dtype=np.int32).reshape(-1, 2))
        rc = L.oracle_attention_pairs(ctypes.byref(p), pr.ctypes.data, pr.shape[0], nt)
    elif f64:
        rc = L.oracle_attention_f64(ctypes.byref(p), nt)
    else:
        rc = L.oracle_attention(ctypes.byref(p), nt)
    if rc != 0:
        raise ValueError("oracle rejected the problem")
    return out, probs


def launch_multihead_attention(qkv, B, S, E, H, causal=False, want_probs=True, nthreads=None):
    """Oracle mirror of the reference launcher on the planar buffer.
    Returns (out [B*S, E], probs [B, H, S, S] or None); raises ValueError
    where the reference aborts."""
    qkv = np.ascontiguousarray(qkv, dtype=np.float32)
    if qkv.size < 3 * B * S * E:
        raise ValueError("qkv too small")
    out = np.zeros((B * S, E), dtype=np.float32)
    probs = np.zeros((B, H, S, S), dtype=np.float32) if want_probs else None
    nt = nthreads if nthreads is not None else min(8, os.cpu_count() or 1)
    rc = _oracle().oracle_launch_multihead_attention(
        qkv.ctypes.data, out.ctypes.data, probs.ctypes.data if probs is not None else None,
        B, S, E, H, int(bool(causal)), nt)
    if rc != 0:
        raise ValueError(f"Bad MHA config: E={E} H={H}")
    return out, probs


def _nt(nthreads):
    return nthreads if nthreads is not None else min(8, os.cpu_count() or 1)


def scaled_dot_product(Q, K, B, S, D, nthreads=None):
    """src/hip_kernels.cpp:455-466 on [B*S, D] inputs -> scores [B*S, S]."""
    Q = np.ascontiguousarray(Q, dtype=np.float32); K = np.ascontiguousarray(K, dtype=np.float32)
    out = np.zeros((B * S, S), dtype=np.float32)
    _oracle().oracle_scaled_dot_product(Q.ctypes.data, K.ctypes.data, out.ctypes.data, B, S, D, _nt(nthreads))
    return out


def softmax_rows(scores, B, S, nthreads=None):
    """src/hip_kernels.cpp:478-502: row softmax of [B*S, S] scores."""
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    out = np.zeros((B * S, S), dtype=np.float32)
    _oracle().oracle_softmax_rows(scores.ctypes.data, out.ctypes.data, B, S, _nt(nthreads))
    return out


def attention_weighted_sum(P, V, B, S, D, nthreads=None):
    """src/hip_kernels.cpp:513-525: [B*S, S] probs times [B*S, D] values."""
    P = np.ascontiguousarray(P, dtype=np.float32); V = np.ascontiguousarray(V, dtype=np.float32)
    out = np.zeros((B * S, D), dtype=np.float32)
    _oracle().oracle_attention_weighted_sum(P.ctypes.data, V.ctypes.data, out.ctypes.data, B, S, D, _nt(nthreads))
    return out


def mha_backward(grad_out, qkv, probs, B, S, E, H, nthreads=None):
    """Restatement of launch_multihead_attention_backward
    (src/hip_kernels.cpp:1159-1272); returns grad_qkv [3*B*S*E].  nthreads
    > 1 spreads the (b, h) pairs over host threads (same result)."""
    g = np.ascontiguousarray(grad_out, dtype=np.float32)
    x = np.ascontiguousarray(qkv, dtype=np.float32)
    p = np.ascontiguousarray(probs, dtype=np.float32)
    out = np.zeros(3 * B * S * E, dtype=np.float32)
    L = _oracle()
    if nthreads is None or nthreads <= 1:
        rc = L.oracle_mha_backward(g.ctypes.data, x.ctypes.data, p.ctypes.data, out.ctypes.data, B, S, E, H)
    else:
        rc = L.oracle_mha_backward_mt(g.ctypes.data, x.ctypes.data, p.ctypes.data, out.ctypes.data, B, S, E, H,
                                      nthreads)
    if rc != 0:
        raise ValueError(f"Bad MHA config: E={E} H={H}")
    return out


def matmul_add_bias(A, Bm, bias, M, N, K):
    """Restatement of launch_matmul_add_bias / launch_matmul
    (src/hip_kernels.cpp:70-154): A [M, N] times B [N, K] (+ bias [K]),
    sequential fused multiply-add over n.  Returns C [M, K] float32."""
    A = np.ascontiguousarray(A, dtype=np.float32).reshape(M, N)
    Bm = np.ascontiguousarray(Bm, dtype=np.float32).reshape(N, K)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32).reshape(K)
    out = np.zeros((M, K), dtype=np.float32)
    _oracle().oracle_matmul_add_bias(A.ctypes.data, Bm.ctypes.data, None if b is None else b.ctypes.data,
                                     out.ctypes.data, M, N, K)
    return out


def planar_qkv(qkv, B, S, E, H):
    """[B, S, H, D] views of the Q, K, V planes of a planar buffer."""
    D = E // H
    planes = qkv.reshape(3, B, S, H, D)
    return planes[0], planes[1], planes[2]


def seeded_planar(seed, B, S, E):
    """The planar d_qkv of one config: 3*B*S*E N(0,1) values, Q then K then V."""
    return fill_normal(seed, 3 * B * S * E)


def seeded_bshd(seed, B, Sq, Sk, H, D):
    """q [B,Sq,H,D], k, v [B,Sk,H,D] from one seeded stream (q, then k, then v)."""
    nq, nk = B * Sq * H * D, B * Sk * H * D
    x = fill_normal(seed, nq + 2 * nk)
    return (x[:nq].reshape(B, Sq, H, D), x[nq:nq + nk].reshape(B, Sk, H, D),
            x[nq + nk:].reshape(B, Sk, H, D))


# ---------------------------------------------------------------- reference
_ref = None


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref_lib():
    """The reference's own src/hip_kernels.cpp built for gfx950 (oracle/_ref).
    Exposes `launch(qkv_ptr, out_ptr, probs_ptr, B, S, E, H)` (C++ symbol
    _Z26launch_multihead_attentionPKfPfS1_iiii).  Import torch first so one
    HIP runtime serves the process."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"{REF_SO} missing: run `make -C oracle ref` where /root/reference exists")
        L = ctypes.CDLL(REF_SO)
        fn = getattr(L, "_Z26launch_multihead_attentionPKfPfS1_iiii")
        fn.restype = None
        fn.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 4
        L.launch = fn
        f = getattr(L, "_Z35launch_multihead_attention_backwardPKfS0_S0_Pfiiii")
        f.restype = None
        f.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 4
        L.backward = f
        for attr, sym, nargs in (("matmul", "_Z13launch_matmulPKfS0_Pfiii", (3, 3)),
                                 ("matmul_add_bias", "_Z22launch_matmul_add_biasPKfS0_S0_Pfiii", (4, 3)),
                                 ("sdp", "_Z25launch_scaled_dot_productPKfS0_Pfiii", (3, 3)),
                                 ("softmax", "_Z14launch_softmaxPKfPfii", (2, 2)),
                                 ("wsum", "_Z29launch_attention_weighted_sumPKfS0_Pfiii", (3, 3))):
            f = getattr(L, sym)
            f.restype = None
            f.argtypes = [ctypes.c_void_p] * nargs[0] + [ctypes.c_int] * nargs[1]
            setattr(L, attr, f)
        _ref = L
    return _ref
