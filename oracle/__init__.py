"""Test infrastructure: CPU restatement of HipGPT's attention forward and the
loader of the reference's own HIP kernels built from its sources.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
package, and only as the checker.  The product (hipgpt_amd/) never imports it.
"""
from .py_oracle import *  # noqa: F401,F403
