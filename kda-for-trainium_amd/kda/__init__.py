"""kda -- MI355X (gfx950) kernels for the NKIBench operator set, one callable per op.

    import kda
    y = kda.ops.silu(x)                  # x: contiguous fp32 GPU tensor

The kernels live in libkda.so (C ABI declared in include/kda.h); ``kda.ops``
binds them through ctypes.  ``kda.harness`` holds the verify.py-style scoring
helpers (relative-L2 across seeds, p50 latency, roofline fraction).
"""
from . import _lib, harness, ops  # noqa: F401

__version__ = "0.1.0"
