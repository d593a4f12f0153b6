"""Per-operator roofline model for the NKIBench operators: what bounds an operator
and how much algorithmic work one call does, from the shapes of its forward()
inputs.  It feeds ``summary_metrics`` and the one-line bottleneck digest that the
reference's verify contract prints per operator (verify.py:48-50, README.md:146-147;
the reference's digests read like "DMA=97% ... HBMrd=117MB HBMwr=117MB",
workspaces/silu/benchmark.csv:2).

Work per call:
- HBM-bound operators: bytes every input is read once and the output written
  once (fp32).
- GEMM-shaped fp32 operators run three bf16 (or fp16) MFMA products per fp32
  product (hi*hi + hi*lo + lo*hi), so their roofline work is the MFMA flops
  issued, 3 x the fp32 product's 2*M*N*K; the fp32-equivalent rate (2*M*N*K / t)
  is reported beside it.
- mamba is HBM-class by bytes but bound by its scan (VALU), which the digest says.

Peaks are MI355X's published figures: HBM 8 TB/s, dense bf16/fp16 MFMA 2.5 PFLOP/s.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Dict, Mapping, Optional, Sequence

PEAK_HBM_BYTES_S = 8.0e12
PEAK_MFMA_FLOP_S = 2.5e15


@dataclass
class Work:
    bound: str                 # "hbm" or "mfma"
    work: float                # bytes (hbm) or MFMA flops issued (mfma) per call
    hbm_bytes: float           # algorithmic HBM bytes per call (inputs read once, output written once)
    useful_flops: float = 0.0  # fp32-equivalent flops of the operator (0 for streaming operators)
    note: str = ""


def _shape(v: Any) -> Sequence[int]:
    s = getattr(v, "shape", None)
    return tuple(int(d) for d in s) if s is not None else ()


def _numel(v: Any) -> int:
    return math.prod(_shape(v)) if _shape(v) else 0


def _mm(m: int, k: int, n: int) -> float:
    return 2.0 * m * k * n


def op_work(op: str, inputs: Mapping[str, Any]) -> Work:
    """Work of one call of `op` on `inputs` (forward()-named arrays or tensors)."""
    arrays = [v for v in inputs.values() if _shape(v)]
    in_bytes = 4.0 * sum(_numel(v) for v in arrays)
    if op == "silu":
        n = _numel(inputs["x"])
        return Work("hbm", 8.0 * n, 8.0 * n)
    if op == "adamw":          # theta, g, m, v read; the new theta written
        n = _numel(inputs["theta"])
        return Work("hbm", 20.0 * n, 20.0 * n)
    if op == "rope_single_freq_apply":
        b = in_bytes + 4.0 * _numel(inputs["x_in"])
        return Work("hbm", b, b)
    if op == "mamba":
        c, m = _shape(inputs["delta"])
        b = in_bytes + 4.0 * c * m
        return Work("hbm", b, b, note="scan-bound (VALU): numpy's float32 exp per (channel, state, step)")
    if op in ("bmm", "bmm_softmax"):
        bb, m, k = _shape(inputs["lhs"])
        n = _shape(inputs["rhs"])[2]
        b = in_bytes + 4.0 * bb * m * n
        return Work("hbm", b, b, useful_flops=_mm(bb * m, k, n))
    if op in ("matmul", "transpose_matmul"):
        ls, rs = _shape(inputs["lhs"]), _shape(inputs["rhs"])
        k, n = rs
        m = ls[1] if op == "transpose_matmul" else ls[0]
        f = _mm(m, k, n)
        return Work("mfma", 3 * f, in_bytes + 4.0 * m * n, useful_flops=f)
    if op in ("rmsnorm_matmul", "add_rmsnorm_matmul", "matmul_add_rmsnorm"):
        m, k = _shape(inputs["x"])
        n = _shape(inputs["w"])[1]
        f = _mm(m, k, n)
        return Work("mfma", 3 * f, in_bytes + 4.0 * m * n, useful_flops=f)
    if op == "lora":
        m, k = _shape(inputs["x"])
        n = _shape(inputs["w"])[1]
        r = _shape(inputs["a"])[1]
        f = _mm(m, k, n) + _mm(m, k, r) + _mm(m, r, n)
        return Work("mfma", 3 * f, in_bytes + 4.0 * m * n, useful_flops=f)
    if op == "swiglu":
        m, k = _shape(inputs["x"])
        n = _shape(inputs["w_up"])[1]
        f = 3 * _mm(m, k, n)
        return Work("mfma", 3 * f, in_bytes + 4.0 * m * k, useful_flops=f)
    if op == "gqa_full":
        b, s, hq, d = _shape(inputs["q"])
        f = 4.0 * b * hq * s * s * d
        return Work("mfma", 3 * f, in_bytes + 4.0 * b * hq * s * d, useful_flops=f)
    raise KeyError(f"no roofline model for operator {op!r}")


def metrics(op: str, inputs: Mapping[str, Any], seconds: float,
            traffic: Optional[Mapping[str, Any]] = None) -> Dict[str, Any]:
    """summary_metrics entries for one call of `seconds`: the bound, achieved rate,
    roofline fraction, algorithmic HBM bytes, and the measured HBM read/write
    bytes when `traffic` (a profile's figures for this operator and shape) is given."""
    w = op_work(op, inputs)
    out: Dict[str, Any] = {"bound": w.bound, "work": w.work, "hbm_bytes_algorithmic": w.hbm_bytes}
    if w.bound == "hbm":
        out.update(achieved=w.work / seconds / 1e9, unit="GB/s", peak=PEAK_HBM_BYTES_S / 1e9,
                   roofline_frac=w.work / seconds / PEAK_HBM_BYTES_S)
    else:
        out.update(achieved=w.work / seconds / 1e12, unit="TFLOP/s", peak=PEAK_MFMA_FLOP_S / 1e12,
                   roofline_frac=w.work / seconds / PEAK_MFMA_FLOP_S)
    if w.useful_flops:
        out["fp32_tflops"] = w.useful_flops / seconds / 1e12
    if w.note:
        out["note"] = w.note
    if traffic:
        out["hbm_read_bytes"] = float(traffic["read_bytes"])
        out["hbm_write_bytes"] = float(traffic["write_bytes"])
        out["hbm_bytes_source"] = str(traffic.get("source", "profile"))
    return out


def _mb(b: float) -> str:
    return f"{b / 1e6:.1f}MB"


def _g(x: float, digits: int = 3) -> str:
    """Significant digits for small values, two decimals (fractions) otherwise."""
    return f"{x:.{digits}g}" if abs(x) < 0.1 else (f"{x:.2f}" if abs(x) < 100 else f"{x:.0f}")


def digest(m: Mapping[str, Any]) -> str:
    """One-line bottleneck digest of a summary_metrics dict."""
    if "bound" not in m:
        return ""
    if m["bound"] == "hbm":
        head = (f"HBM {_g(m['achieved'] / 1e3)} TB/s = {_g(m['roofline_frac'])} of "
                f"{m['peak'] / 1e3:.0f} TB/s")
    else:
        head = (f"MFMA {_g(m['achieved'])} TFLOP/s issued = {_g(m['roofline_frac'])} of "
                f"{m['peak'] / 1e3:.1f} PFLOP/s")
    parts = [head]
    if "fp32_tflops" in m and m["bound"] == "mfma":
        parts.append(f"fp32-equivalent {_g(m['fp32_tflops'])} TFLOP/s")
    if "hbm_read_bytes" in m:
        parts.append(f"HBMrd={_mb(m['hbm_read_bytes'])} HBMwr={_mb(m['hbm_write_bytes'])} "
                     f"(algorithmic {_mb(m['hbm_bytes_algorithmic'])})")
    else:
        parts.append(f"HBM algorithmic {_mb(m['hbm_bytes_algorithmic'])}")
    if m.get("note"):
        parts.append(m["note"])
    return "; ".join(parts)
