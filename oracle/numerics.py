"""bf16 rounding, two-limb bf16 split and relative-L2 -- oracle helpers.

Test infrastructure only (see oracle/__init__.py).
"""
from __future__ import annotations

import numpy as np


def to_bf16_rne(x) -> np.ndarray:
    """fp32 -> bf16 round-to-nearest-even, returned as fp32 values.

    Follows workspaces/matmul/runs/offline_bf16_split_sim.py:94-114: keep the
    top 16 bits of the fp32 pattern after adding ``0x7FFF + lsb`` (lsb = bit 16).
    NaN inputs are kept NaN (quiet) rather than being rounded through.
    """
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)) << np.uint64(16)
    out = (r & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32)
    nan = np.isnan(x)
    if np.any(nan):
        out = np.where(nan, np.float32(np.nan), out)
    return out


def split_bf16x2(x):
    """x ~= hi + lo with hi, lo bf16-valued (workspaces/matmul/runs/offline_bf16_split_sim.py:117-122)."""
    x = np.asarray(x, dtype=np.float32)
    hi = to_bf16_rne(x)
    lo = to_bf16_rne((x - hi).astype(np.float32))
    return hi, lo


def rel_l2(kernel_out, reference_out) -> float:
    """||k - r||_2 / ||r||_2, float64 norms (workspaces/matmul/runs/offline_bf16_split_sim.py:210-214)."""
    k = np.asarray(kernel_out, dtype=np.float64).ravel()
    r = np.asarray(reference_out, dtype=np.float64).ravel()
    den = np.linalg.norm(r)
    num = np.linalg.norm(k - r)
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return float(num / den)
