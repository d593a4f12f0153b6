"""Seeded input draws for every case -- oracle.

Test infrastructure only (see oracle/__init__.py).

Two families:

* NKIBench cases (the reference's fp32 operator shapes).  Draw model of the
  reference: ``np.random.seed(seed)`` once, then ``np.random.normal`` for each
  forward() parameter in order, cast to float32; python-float parameters (eps)
  draw nothing (adapter/nkibench_case.py:142-155; e.g.
  workspaces/add_rmsnorm_matmul/runs/offline_bf16_split_sim.py:81-94).  The
  scale is N(0,1) except mamba (N(0, 0.05): workspaces/mamba/docs/draft-phase1.md:93-96)
  and AdamW's v = |N(0,1)| (workspaces/adamw/docs/plan-phase1.md:233-234).
  Unlike the reference's adapter, each seed really draws different inputs.
* Graded configurations (SiLU fp32, RMSNorm->matmul bf16, SwiGLU bf16, AdamW
  fp32, causal GQA bf16), and the two residual RMSNorm variants at the
  RMSNorm->matmul shape in bf16.  Distributions as specified per configuration; the
  generator is ``np.random.default_rng(seed)`` (float32 ``standard_normal``,
  scaled), chosen over the legacy generator for speed at 10^8-element sizes.
  bf16 inputs are drawn in fp32 and rounded once to bf16 (RNE); the GPU and the
  oracle receive the same bf16 values.

Every draw accepts ``dims`` overrides so tests can run the same case at small
sizes.
"""
from __future__ import annotations

from typing import Dict, Optional

import numpy as np

from .numerics import to_bf16_rne

F32 = np.float32

# forward() parameter names (and kernel argument order) per case.
PARAMS = {
    "silu": ["x"],
    "adamw": ["theta", "g", "m", "v"],
    "rope_single_freq_apply": ["x_in", "cos", "sin"],
    "mamba": ["delta", "u", "a", "b", "c"],
    "matmul": ["lhs", "rhs"],
    "transpose_matmul": ["lhs", "rhs"],
    "bmm": ["lhs", "rhs"],
    "bmm_softmax": ["lhs", "rhs"],
    "lora": ["x", "w", "a", "b"],
    "rmsnorm_matmul": ["x", "w"],
    "add_rmsnorm_matmul": ["x", "w", "eps", "z", "g"],
    "matmul_add_rmsnorm": ["x", "w", "eps", "z", "g"],
    "swiglu": ["x", "w_up", "w_down", "w_gate"],
    "gqa_full": ["q", "k", "v"],
    # graded configurations
    "silu_cfg": ["x"],
    "rmsnorm_matmul_cfg": ["x", "gamma", "w", "eps"],
    "add_rmsnorm_matmul_cfg": ["x", "w", "eps", "z", "g"],
    "matmul_add_rmsnorm_cfg": ["x", "w", "eps", "z", "g"],
    "swiglu_cfg": ["x", "w_up", "w_down", "w_gate"],
    "adamw_cfg": ["param", "grad", "m", "v"],
    "gqa_cfg": ["q", "k", "v"],
}

# Full sizes (the reference's NKIBench shapes, prompts/_gen_prompts.py:17-256,
# and the graded configuration shapes).
DIMS = {
    "silu": dict(M=4096, N=7168),
    "adamw": dict(M=10944, N=2048),
    "rope_single_freq_apply": dict(D=128, S=262144),
    "mamba": dict(C=256, M=7168, S=16),
    "matmul": dict(M=4096, K=5120, N=12288),
    "transpose_matmul": dict(M=4096, K=2048, N=10944),
    "bmm": dict(B=16, M=4096, K=64, N=4096),
    "bmm_softmax": dict(B=16, M=4096, K=64, N=4096),
    "lora": dict(M=4096, K=5120, N=12288, R=128),
    "rmsnorm_matmul": dict(M=4096, K=1024, N=2048),
    "add_rmsnorm_matmul": dict(M=4096, K=1024, N=2048),
    "matmul_add_rmsnorm": dict(M=4096, K=2048, N=2048),
    "swiglu": dict(M=4096, K=1024, N=3072),
    "gqa_full": dict(B=1, S=4096, HQ=16, HKV=8, D=128),
    "silu_cfg": dict(M=2048, N=8192),
    "rmsnorm_matmul_cfg": dict(M=4096, K=4096, N=11008),
    "add_rmsnorm_matmul_cfg": dict(M=4096, K=4096, N=11008),
    "matmul_add_rmsnorm_cfg": dict(M=4096, K=4096, N=11008),
    "swiglu_cfg": dict(M=2048, K=4096, F=14336),
    "adamw_cfg": dict(N=1 << 27),
    "gqa_cfg": dict(B=4, S=4096, HQ=32, HKV=8, D=128),
}

EPS = {"add_rmsnorm_matmul": 1e-5, "matmul_add_rmsnorm": 1e-5, "rmsnorm_matmul_cfg": 1e-6,
       "add_rmsnorm_matmul_cfg": 1e-6, "matmul_add_rmsnorm_cfg": 1e-6}

# AdamW configuration hyper-parameters.
ADAMW_CFG = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, step=10)


def _legacy(seed: int, shapes, scale: float = 1.0):
    np.random.seed(seed)
    return [np.random.normal(loc=0.0, scale=scale, size=s).astype(F32) for s in shapes]


def _rng_normal(rng, shape, mean=0.0, std=1.0):
    z = rng.standard_normal(size=shape, dtype=F32)
    if std != 1.0:
        z *= F32(std)
    if mean != 0.0:
        z += F32(mean)
    return z


def draw(case: str, seed: int, dims: Optional[Dict[str, int]] = None) -> Dict[str, object]:
    """Inputs of `case` for `seed`, keyed by forward() parameter names."""
    d = dict(DIMS[case])
    if dims:
        d.update(dims)
    if case == "silu":
        (x,) = _legacy(seed, [(d["M"], d["N"])])
        return {"x": x}
    if case == "adamw":
        shp = (d["M"], d["N"])
        theta, g, m, v = _legacy(seed, [shp] * 4)
        return {"theta": theta, "g": g, "m": m, "v": np.abs(v)}
    if case == "rope_single_freq_apply":
        x_in, cos, sin = _legacy(seed, [(d["D"], d["S"]), (d["D"] // 2, d["S"]), (d["D"] // 2, d["S"])])
        return {"x_in": x_in, "cos": cos, "sin": sin}
    if case == "mamba":
        C, M, S = d["C"], d["M"], d["S"]
        delta, u, a, b, c = _legacy(seed, [(C, M), (C, M), (C, S), (S, M), (S, M)], scale=0.05)
        return {"delta": delta, "u": u, "a": a, "b": b, "c": c}
    if case == "matmul":
        lhs, rhs = _legacy(seed, [(d["M"], d["K"]), (d["K"], d["N"])])
        return {"lhs": lhs, "rhs": rhs}
    if case == "transpose_matmul":
        lhs, rhs = _legacy(seed, [(d["K"], d["M"]), (d["K"], d["N"])])
        return {"lhs": lhs, "rhs": rhs}
    if case in ("bmm", "bmm_softmax"):
        lhs, rhs = _legacy(seed, [(d["B"], d["M"], d["K"]), (d["B"], d["K"], d["N"])])
        return {"lhs": lhs, "rhs": rhs}
    if case == "lora":
        x, w, a, b = _legacy(seed, [(d["M"], d["K"]), (d["K"], d["N"]), (d["K"], d["R"]), (d["R"], d["N"])])
        return {"x": x, "w": w, "a": a, "b": b}
    if case == "rmsnorm_matmul":
        x, w = _legacy(seed, [(d["M"], d["K"]), (d["K"], d["N"])])
        return {"x": x, "w": w}
    if case == "add_rmsnorm_matmul":
        M, K, N = d["M"], d["K"], d["N"]
        x, w, z, g = _legacy(seed, [(M, K), (K, N), (M, K), (K,)])
        return {"x": x, "w": w, "eps": EPS[case], "z": z, "g": g}
    if case == "matmul_add_rmsnorm":
        M, K, N = d["M"], d["K"], d["N"]
        x, w, z, g = _legacy(seed, [(M, K), (K, N), (M, N), (N,)])
        return {"x": x, "w": w, "eps": EPS[case], "z": z, "g": g}
    if case == "swiglu":
        M, K, N = d["M"], d["K"], d["N"]
        x, w_up, w_down, w_gate = _legacy(seed, [(M, K), (K, N), (N, K), (K, N)])
        return {"x": x, "w_up": w_up, "w_down": w_down, "w_gate": w_gate}
    if case == "gqa_full":
        B, S, HQ, HKV, D = d["B"], d["S"], d["HQ"], d["HKV"], d["D"]
        q, k, v = _legacy(seed, [(B, S, HQ, D), (B, S, HKV, D), (B, S, HKV, D)])
        return {"q": q, "k": k, "v": v}

    rng = np.random.default_rng(seed)
    if case == "silu_cfg":
        return {"x": _rng_normal(rng, (d["M"], d["N"]))}
    if case == "rmsnorm_matmul_cfg":
        M, K, N = d["M"], d["K"], d["N"]
        x = to_bf16_rne(_rng_normal(rng, (M, K)))
        gamma = to_bf16_rne(_rng_normal(rng, (K,), mean=1.0, std=0.1))
        w = to_bf16_rne(_rng_normal(rng, (K, N), std=0.02))
        return {"x": x, "gamma": gamma, "w": w, "eps": EPS[case]}
    if case == "add_rmsnorm_matmul_cfg":
        M, K, N = d["M"], d["K"], d["N"]
        x = to_bf16_rne(_rng_normal(rng, (M, K)))
        z = to_bf16_rne(_rng_normal(rng, (M, K)))
        g = to_bf16_rne(_rng_normal(rng, (K,), mean=1.0, std=0.1))
        w = to_bf16_rne(_rng_normal(rng, (K, N), std=0.02))
        return {"x": x, "w": w, "eps": EPS[case], "z": z, "g": g}
    if case == "matmul_add_rmsnorm_cfg":
        M, K, N = d["M"], d["K"], d["N"]
        x = to_bf16_rne(_rng_normal(rng, (M, K)))
        w = to_bf16_rne(_rng_normal(rng, (K, N), std=0.02))
        z = to_bf16_rne(_rng_normal(rng, (M, N)))
        g = to_bf16_rne(_rng_normal(rng, (N,), mean=1.0, std=0.1))
        return {"x": x, "w": w, "eps": EPS[case], "z": z, "g": g}
    if case == "swiglu_cfg":
        M, K, F = d["M"], d["K"], d["F"]
        x = to_bf16_rne(_rng_normal(rng, (M, K)))
        w_gate = to_bf16_rne(_rng_normal(rng, (K, F), std=0.02))
        w_up = to_bf16_rne(_rng_normal(rng, (K, F), std=0.02))
        w_down = to_bf16_rne(_rng_normal(rng, (F, K), std=0.02))
        return {"x": x, "w_up": w_up, "w_down": w_down, "w_gate": w_gate}
    if case == "adamw_cfg":
        n = d["N"]
        param = _rng_normal(rng, (n,), std=0.02)
        grad = _rng_normal(rng, (n,), std=1e-3)
        m = _rng_normal(rng, (n,), std=1e-4)
        v = np.abs(_rng_normal(rng, (n,), std=1e-6))
        return {"param": param, "grad": grad, "m": m, "v": v}
    if case == "gqa_cfg":
        B, S, HQ, HKV, D = d["B"], d["S"], d["HQ"], d["HKV"], d["D"]
        q = to_bf16_rne(_rng_normal(rng, (B, S, HQ, D)))
        k = to_bf16_rne(_rng_normal(rng, (B, S, HKV, D)))
        v = to_bf16_rne(_rng_normal(rng, (B, S, HKV, D)))
        return {"q": q, "k": k, "v": v}
    raise KeyError(f"unknown case {case!r}")
