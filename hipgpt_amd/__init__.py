"""hipgpt_amd -- MI355X (gfx950) attention forward for HipGPT.

The product is libhipgpt_attn.so (hand-written HIP, C ABI in include/).  This
package builds nothing at import time; it binds the in-tree library.
``hipgpt_amd.attention`` (needs torch) is the tensor-level host interface.
"""
from ._lib import LIB_PATH, HipgptError, lib  # noqa: F401

__all__ = ["LIB_PATH", "HipgptError", "lib"]
