"""ctypes binding of libhipgpt_attn.so (include/hip_kernels.h, include/hipgpt_attn.h).

The shared library is built in-tree (``make -C hipgpt_amd/csrc``) and loaded
from this package directory.  There is no fallback: a missing or stale build
raises, so no caller can silently run anything but the HIP kernels.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhipgpt_attn.so")

# Status codes of include/hipgpt_attn.h.
OK = 0
ERR_INVALID = -1
ERR_UNSUPPORTED = -2
ERR_LAUNCH = -3
ERR_WORKSPACE = -4
ERR_SCRATCH = -5

F32 = 0
BF16 = 1

QKV_ROWS = 0
QKV_PLANAR = 1

# Entry points declared in include/*.h, with their ctypes signatures.
_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_f = ctypes.c_float

SIGNATURES = {
    "hipgpt_attn_strerror": (ctypes.c_char_p, [_int]),
    "hipgpt_launch_multihead_attention": (None, [_vp, _vp, _vp, _int, _int, _int, _int]),
    "hipgpt_launch_scaled_dot_product": (None, [_vp, _vp, _vp, _int, _int, _int]),
    "hipgpt_launch_softmax": (None, [_vp, _vp, _int, _int]),
    "hipgpt_launch_attention_weighted_sum": (None, [_vp, _vp, _vp, _int, _int, _int]),
    "hipgpt_launch_multihead_attention_backward": (None, [_vp, _vp, _vp, _vp, _int, _int, _int, _int]),
    "hipgpt_attn_bwd_workspace_bytes": (ctypes.c_size_t, [_int, _int, _int]),
    "hipgpt_attn_bwd_qkv_planar": (
        _int, [_vp, _vp, _vp, _vp, _int, _int, _int, _int, _int, _vp, ctypes.c_size_t, _vp]),
    "hipgpt_attn_bwd_qkv_planar_noalloc": (_int, [_vp, _vp, _vp, _vp, _int, _int, _int, _int, _int, _vp]),
    "hipgpt_attn_qkv_planar": (_int, [_vp, _vp, _vp, _int, _int, _int, _int, _int, _vp]),
    "hipgpt_attn_fwd_lse_qkv_planar": (_int, [_vp, _vp, _vp, _int, _int, _int, _int, _int, _vp]),
    "hipgpt_attn_bwd_lse_qkv_planar": (
        _int, [_vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _int, _vp, ctypes.c_size_t, _vp]),
    "hipgpt_attn_fwd": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _int]
        + [_i64] * 12
        + [_f, _int, _int, _vp],
    ),
    "hipgpt_attn_decode_kvcache": (
        _int,
        [_vp] * 7 + [_int] * 4 + [_i64] * 11 + [_f, _int, _int, _vp, ctypes.c_size_t, _vp],
    ),
    "hipgpt_launch_matmul": (None, [_vp, _vp, _vp, _int, _int, _int]),
    "hipgpt_launch_matmul_add_bias": (None, [_vp, _vp, _vp, _vp, _int, _int, _int]),
    "hipgpt_gemm_bias": (
        _int, [_vp, _vp, _vp, _vp, _int, _int, _int, _i64, _i64, _i64, _int, _i64, _int, _vp]),
    "hipgpt_qkv_projection": (_int, [_vp, _vp, _vp, _vp, _int, _int, _int, _int, _vp]),
    "hipgpt_attn_wait_expired": (_int, [ctypes.POINTER(ctypes.c_uint), _int]),
    "hipgpt_attn_decode_default_splits": (_int, [_int, _int, _int]),
    "hipgpt_attn_decode_workspace_bytes": (ctypes.c_size_t, [_int, _int, _int, _int]),
    "hipgpt_attn_decode": (
        _int,
        [_vp, _vp, _vp, _vp, _int, _int, _int, _int]
        + [_i64] * 10
        + [_f, _int, _vp, ctypes.c_size_t, _vp],
    ),
}
# The drop-in C++ symbols (HipGPT include/hip_kernels.h:39-46).
CXX_LAUNCH_SYMBOL = "_Z26launch_multihead_attentionPKfPfS1_iiii"
CXX_HELPER_SYMBOLS = {
    "launch_scaled_dot_product": "_Z25launch_scaled_dot_productPKfS0_Pfiii",
    "launch_softmax": "_Z14launch_softmaxPKfPfii",
    "launch_attention_weighted_sum": "_Z29launch_attention_weighted_sumPKfS0_Pfiii",
    "launch_multihead_attention_backward": "_Z35launch_multihead_attention_backwardPKfS0_S0_Pfiiii",
    "launch_matmul": "_Z13launch_matmulPKfS0_Pfiii",
    "launch_matmul_add_bias": "_Z22launch_matmul_add_biasPKfS0_S0_Pfiii",
}

_lib = None
_lock = threading.Lock()


class HipgptError(RuntimeError):
    """A non-OK status from the library."""

    def __init__(self, status: int, what: str = ""):
        self.status = status
        msg = lib().hipgpt_attn_strerror(status).decode()
        super().__init__(f"{what}: {msg} (status {status})" if what else msg)


def lib() -> ctypes.CDLL:
    """Load (once) and return the library with typed entry points."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `make -C hipgpt_amd/csrc` "
                    "(or __graft_entry__.build())"
                )
            handle = ctypes.CDLL(LIB_PATH)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            cxx = getattr(handle, CXX_LAUNCH_SYMBOL)
            cxx.restype = None
            cxx.argtypes = SIGNATURES["hipgpt_launch_multihead_attention"][1]
            _lib = handle
    return _lib


def wait_expired(clear: bool = True) -> int:
    """Bounded LDS-flag waits that ran out on the current device since the
    last clear (hipgpt_attn_wait_expired); zero in a correct run."""
    n = ctypes.c_uint(0)
    check(lib().hipgpt_attn_wait_expired(ctypes.byref(n), 1 if clear else 0), "hipgpt_attn_wait_expired")
    return int(n.value)


def check(status: int, what: str = "") -> None:
    if status != OK:
        raise HipgptError(status, what)
