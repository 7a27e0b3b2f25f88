"""CPU tests of the C-ABI library: it loads, exports every entry point the
public headers declare (plus the drop-in C++ symbol), and rejects bad
arguments before touching the GPU -- including the reference's abort on a
bad head configuration (src/hip_kernels.cpp:410-413)."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

from hipgpt_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("hip_kernels.h", "hipgpt_attn.h")]


def declared_functions(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return set(re.findall(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\([^;{]*\)\s*;", text))


def test_headers_declare_expected_entry_points():
    c_api = declared_functions(HEADERS[1])
    assert set(_lib.SIGNATURES) == c_api
    assert declared_functions(HEADERS[0]) == {"launch_multihead_attention", "launch_scaled_dot_product",
                                               "launch_softmax", "launch_attention_weighted_sum",
                                               "launch_multihead_attention_backward", "launch_matmul",
                                               "launch_matmul_add_bias"}


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in declared_functions(HEADERS[1]):
        assert hasattr(L, name), name
    # HipGPT's C++ launcher, exact mangled name (include/hip_kernels.h:39-43)
    assert hasattr(L, "_Z26launch_multihead_attentionPKfPfS1_iiii")
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True)
    assert " T _Z26launch_multihead_attentionPKfPfS1_iiii" in out.stdout
    for sym in _lib.CXX_HELPER_SYMBOLS.values():  # include/hip_kernels.h:44-46, exact C++ names
        assert f" T {sym}" in out.stdout, sym


def test_no_undefined_library_symbols():
    """Every symbol of the library's own namespace is defined (a kernel whose
    host launch stub the compiler dropped shows up here as undefined, and the
    library would fail to load on the GPU box)."""
    out = subprocess.run(["nm", "-u", _lib.LIB_PATH], capture_output=True, text=True).stdout
    missing = [ln.split()[-1] for ln in out.splitlines() if "6hipgpt" in ln]
    assert not missing, missing


def test_strerror_and_host_validation():
    L = _lib.lib()
    assert L.hipgpt_attn_strerror(0) == b"ok"
    assert b"invalid" in L.hipgpt_attn_strerror(_lib.ERR_INVALID)
    z = [0] * 12
    # null pointers, bad sizes, causal with Sk < Sq, bad dtype: all rejected host-side
    assert L.hipgpt_attn_fwd(None, None, None, None, None, 1, 1, 1, 1, 32, *z, -1.0, 0, 0, None) == _lib.ERR_INVALID
    p = 4096  # any non-null value: validation fails before any dereference
    assert L.hipgpt_attn_fwd(p, p, p, p, None, 1, 1, 0, 1, 32, *z, -1.0, 0, 0, None) == _lib.ERR_INVALID
    assert L.hipgpt_attn_fwd(p, p, p, p, None, 1, 1, 8, 4, 32, *z, -1.0, 1, 0, None) == _lib.ERR_INVALID
    assert L.hipgpt_attn_fwd(p, p, p, p, None, 1, 1, 8, 8, 32, *z, -1.0, 0, 7, None) == _lib.ERR_INVALID
    assert L.hipgpt_attn_qkv_planar(p, p, None, 1, 4, 63, 2, 0, None) == _lib.ERR_INVALID
    assert L.hipgpt_attn_decode(None, None, None, None, 1, 1, 8, 64, *([0] * 10), -1.0, 1, None, 0, None) == _lib.ERR_INVALID
    # unsupported decode head dim, and a missing workspace for several splits
    assert L.hipgpt_attn_decode(p, p, p, p, 1, 1, 8, 48, *([0] * 10), -1.0, 1, None, 0, None) == _lib.ERR_UNSUPPORTED
    assert L.hipgpt_attn_decode(p, p, p, p, 1, 1, 512, 64, *([0] * 10), -1.0, 4, None, 0, None) == _lib.ERR_WORKSPACE
    assert L.hipgpt_attn_decode_workspace_bytes(2, 3, 64, 4) == 2 * 3 * 4 * 66 * 4
    assert L.hipgpt_attn_decode_workspace_bytes(2, 3, 64, 1) == 0
    # one split once B*H alone fills the chip (c5), more for small batches
    assert L.hipgpt_attn_decode_default_splits(64, 12, 2048) == 1
    assert L.hipgpt_attn_decode_default_splits(1, 12, 32768) >= 16
    assert L.hipgpt_attn_decode_default_splits(4, 12, 200) == 1  # no split below 128 keys
    assert L.hipgpt_attn_bwd_workspace_bytes(2, 8, 3) == 2 * 3 * 8 * 4
    assert L.hipgpt_attn_bwd_qkv_planar(p, p, p, p, 1, 8, 64, 2, 0, None, 0, None) == _lib.ERR_WORKSPACE
    assert L.hipgpt_attn_bwd_qkv_planar(p, p, p, p, 1, 8, 63, 2, 0, p, 1 << 20, None) == _lib.ERR_INVALID
    # probs-free training pair: null lse/out, bad split, D not a multiple of 4 or above 256, unaligned,
    # missing workspace (head dims other than 32 / 64)
    fl, bl = L.hipgpt_attn_fwd_lse_qkv_planar, L.hipgpt_attn_bwd_lse_qkv_planar
    assert fl(p, p, None, 1, 8, 64, 2, 1, None) == _lib.ERR_INVALID
    assert fl(p, p, p, 1, 8, 63, 2, 1, None) == _lib.ERR_INVALID
    assert fl(p, p, p, 1, 8, 100, 2, 1, None) == _lib.ERR_UNSUPPORTED   # D = 50
    assert fl(p, p, p, 1, 8, 520, 2, 1, None) == _lib.ERR_UNSUPPORTED   # D = 260
    assert fl(p + 4, p, p, 1, 8, 64, 2, 1, None) == _lib.ERR_UNSUPPORTED  # qkv not 16-byte aligned
    assert bl(p, p, None, p, p, 1, 8, 64, 2, 1, p, 1 << 20, None) == _lib.ERR_INVALID
    assert bl(p, p, p, None, p, 1, 8, 64, 2, 1, p, 1 << 20, None) == _lib.ERR_INVALID
    assert bl(p, p, p, p, p, 1, 8, 100, 2, 1, p, 1 << 20, None) == _lib.ERR_UNSUPPORTED  # D = 50
    assert bl(p, p, p, p, p, 1, 8, 256, 2, 1, None, 0, None) == _lib.ERR_WORKSPACE  # D = 128
    assert bl(p, p, p, p, p, 1, 8, 256, 2, 1, p, 2 * 8 * 4 - 4, None) == _lib.ERR_WORKSPACE
    # KV-cache decode: null lens / caches, bad sizes, unsupported D, missing workspace
    kvc = L.hipgpt_attn_decode_kvcache
    z11 = [0] * 11
    assert kvc(p, p, p, p, p, None, p, 2, 2, 64, 16, *z11, -1.0, 1, 1, None, 0, None) == _lib.ERR_INVALID
    assert kvc(p, p, p, None, p, p, p, 2, 2, 64, 16, *z11, -1.0, 1, 1, None, 0, None) == _lib.ERR_INVALID
    assert kvc(p, p, p, p, p, p, p, 2, 2, 64, 0, *z11, -1.0, 1, 1, None, 0, None) == _lib.ERR_INVALID
    assert kvc(p, p, p, p, p, p, p, 2, 2, 48, 16, *z11, -1.0, 1, 1, None, 0, None) == _lib.ERR_UNSUPPORTED
    assert kvc(p, p, p, p, p, p, p, 2, 2, 64, 4096, *z11, -1.0, 8, 1, None, 0, None) == _lib.ERR_WORKSPACE
    # GEMM: bad sizes, strides, segment split and dtype are rejected host-side
    gemm = L.hipgpt_gemm_bias
    assert gemm(p, p, None, None, 4, 4, 4, 4, 4, 4, 4, 0, 0, None) == _lib.ERR_INVALID   # no output
    assert gemm(p, p, None, p, 0, 4, 4, 4, 4, 4, 4, 0, 0, None) == _lib.ERR_INVALID      # M = 0
    assert gemm(p, p, None, p, 4, 4, -1, 4, 4, 4, 4, 0, 0, None) == _lib.ERR_INVALID     # K < 0
    assert gemm(None, p, None, p, 4, 4, 4, 4, 4, 4, 4, 0, 0, None) == _lib.ERR_INVALID   # no A with K > 0
    assert gemm(p, p, None, p, 4, 4, 8, 4, 4, 4, 4, 0, 0, None) == _lib.ERR_INVALID      # lda < K
    assert gemm(p, p, None, p, 4, 8, 4, 4, 4, 8, 8, 0, 0, None) == _lib.ERR_INVALID      # ldw < N
    assert gemm(p, p, None, p, 4, 8, 4, 4, 8, 8, 9, 0, 0, None) == _lib.ERR_INVALID      # seg_w > N
    assert gemm(p, p, None, p, 4, 8, 4, 4, 8, 2, 4, 0, 0, None) == _lib.ERR_INVALID      # ldc < seg_w
    assert gemm(p, p, None, p, 4, 8, 4, 4, 8, 8, 8, -1, 0, None) == _lib.ERR_INVALID     # seg_stride < 0
    assert gemm(p, p, None, p, 4, 8, 4, 4, 8, 8, 8, 0, 5, None) == _lib.ERR_INVALID      # dtype
    assert L.hipgpt_qkv_projection(p, p, p, p, 4, 8, 2, 0, None) == _lib.ERR_INVALID     # layout
    assert L.hipgpt_qkv_projection(p, p, p, p, 0, 8, 0, 0, None) == _lib.ERR_INVALID     # T = 0


@pytest.mark.parametrize("sym", ["hipgpt_launch_multihead_attention", "_Z26launch_multihead_attentionPKfPfS1_iiii",
                                 "hipgpt_launch_multihead_attention_backward",
                                 "_Z35launch_multihead_attention_backwardPKfS0_S0_Pfiiii"])
@pytest.mark.parametrize("E,H", [(63, 2), (64, 0), (64, -1)])
def test_bad_config_aborts_like_reference(sym, E, H):
    nptr = 4 if "backward" in sym else 3
    code = (
        "import ctypes,sys; L=ctypes.CDLL(sys.argv[1]); f=getattr(L, sys.argv[2]);"
        f"f.argtypes=[ctypes.c_void_p]*{nptr}+[ctypes.c_int]*4;"
        f"f(*([None]*{nptr}),2,4,{E},{H})"
    )
    r = subprocess.run([sys.executable, "-c", code, _lib.LIB_PATH, sym], capture_output=True, text=True)
    assert r.returncode == -6, r  # SIGABRT
    assert f"Bad MHA config: E={E} H={H}" in r.stderr
