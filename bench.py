#!/usr/bin/env python3
"""Benchmark of the five graded operator configurations on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--iters I] [--no-cpu]

Metric: p50 latency per op + % of HBM/MFMA roofline; geomean speedup vs host
numpy.  For each configuration the GPU kernel is timed with HIP events on the
stream it is launched on (p50 over --iters reps after warmup; memory-bound ops
rotate buffer sets larger than the 256 MB Infinity Cache), and the numpy
reference forward is timed on this host's CPU (bounded samples, scaled).  The
"step" of the driver contract is one pass over the five operators; K steps are
timed between two device synchronisations.

Prints exactly one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "kda-for-trainium_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "p50 latency per op + % of HBM/MFMA roofline; geomean speedup vs host numpy"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ----------------------------------------------------------------- configurations
# Algorithmic work per call (bytes for HBM-bound ops, flops for MFMA-bound ops).
CONFIGS = {
    "silu": dict(desc="SiLU fp32 x[2048,8192]", dtype="fp32", bound="hbm",
                 work=2048 * 8192 * 8, kernels=["silu_vec_kernel"]),
    "rmsnorm_matmul": dict(desc="RMSNorm->matmul bf16 x[4096,4096] W[4096,11008]", dtype="bf16",
                           bound="mfma", work=2 * 4096 * 4096 * 11008,
                           kernels=["rms_prep_kernel", "gemm_bf16_kernel<256,256,1,kRowScale>"]),
    "swiglu": dict(desc="SwiGLU bf16 x[2048,4096] Wg/Wu[4096,14336] Wd[14336,4096]", dtype="bf16",
                   bound="mfma", work=6 * 2048 * 4096 * 14336,
                   kernels=["gemm_bf16_kernel<256,128,2,kSwiGLU>", "gemm_bf16_kernel<256,128,1,kStore>"]),
    "adamw": dict(desc="AdamW fp32 n=2^27 in-place step 10", dtype="fp32", bound="hbm",
                  work=28 * (1 << 27), kernels=["adamw_vec_kernel<true>"]),
    "gqa": dict(desc="causal GQA bf16 B4 S4096 Hq32 Hkv8 D128", dtype="bf16", bound="mfma",
                work=4 * 4 * 32 * 4096 * 4096 * 128 // 2, kernels=["gqa_fwd_kernel<true>"]),
}


def make_gpu_case(name, dev, seed=0):
    """Synthetic inputs of each configuration's distribution, drawn on the GPU.
    Returns (fn(i) running one call on rotation slot i, keep-alive list)."""
    import torch
    from kda import ops
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    BF = torch.bfloat16

    def normal(shape, std=1.0, mean=0.0, dtype=torch.float32):
        t = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
        if std != 1.0:
            t.mul_(std)
        if mean != 0.0:
            t.add_(mean)
        return t.to(dtype)

    if name == "silu":
        sets = [(normal((2048, 8192)), torch.empty(2048, 8192, device=dev)) for _ in range(4)]
        return (lambda i: ops.silu(sets[i % 4][0], out=sets[i % 4][1])), sets
    if name == "rmsnorm_matmul":
        x = normal((4096, 4096), dtype=BF)
        gamma = normal((4096,), std=0.1, mean=1.0, dtype=BF)
        w = normal((4096, 11008), std=0.02, dtype=BF)
        return (lambda i: ops.rmsnorm_matmul(x, w, gamma=gamma, eps=1e-6)), [x, gamma, w]
    if name == "swiglu":
        x = normal((2048, 4096), dtype=BF)
        wg = normal((4096, 14336), std=0.02, dtype=BF)
        wu = normal((4096, 14336), std=0.02, dtype=BF)
        wd = normal((14336, 4096), std=0.02, dtype=BF)
        h = torch.empty(2048, 14336, device=dev, dtype=BF)
        return (lambda i: ops.swiglu(x, wu, wd, wg, h_workspace=h)), [x, wg, wu, wd, h]
    if name == "adamw":
        n = 1 << 27
        p, gr, m = normal((n,), std=0.02), normal((n,), std=1e-3), normal((n,), std=1e-4)
        v = normal((n,), std=1e-6).abs_()
        hp = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, step=10)
        return (lambda i: ops.adamw_step_(p, gr, m, v, **hp)), [p, gr, m, v]
    if name == "gqa":
        q = normal((4, 4096, 32, 128), dtype=BF)
        k = normal((4, 4096, 8, 128), dtype=BF)
        v = normal((4, 4096, 8, 128), dtype=BF)
        return (lambda i: ops.gqa(q, k, v, causal=True)), [q, k, v]
    raise KeyError(name)


# ----------------------------------------------------------------- CPU baseline

def cpu_baseline(name, reps=3):
    """Times the numpy reference forward (the oracle) on this host; bounded sample,
    scaled linearly to the full configuration.  Returns (ms, sample description)."""
    import numpy as np
    from oracle import inputs as oi
    from oracle import ops as oo

    def timed(fn, reps=reps):
        fn()  # warmup
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2] * 1e3

    if name == "silu":
        d = oi.draw("silu_cfg", 0)
        return timed(lambda: oo.silu(d["x"])), "full x[2048,8192]"
    if name == "rmsnorm_matmul":
        d = oi.draw("rmsnorm_matmul_cfg", 0)
        return timed(lambda: oo.rmsnorm_matmul_gamma(**d)), "full (fp32 numpy on bf16 values)"
    if name == "swiglu":
        d = oi.draw("swiglu_cfg", 0)
        return timed(lambda: oo.swiglu(**d)), "full (fp32 numpy on bf16 values)"
    if name == "adamw":
        frac = 8
        d = oi.draw("adamw_cfg", 0, dims=dict(N=(1 << 27) // frac))
        ms = timed(lambda: oo.adamw_step(d["param"], d["grad"], d["m"], d["v"], **oi.ADAMW_CFG))
        return ms * frac, f"n=2^24 (1/{frac} of the buffer), scaled x{frac}"
    if name == "gqa":
        d = oi.draw("gqa_cfg", 0, dims=dict(B=1, HQ=4, HKV=1))
        ms = timed(lambda: oo.gqa(d["q"], d["k"], d["v"], causal=True), reps=1)
        return ms * 32, "one (batch, kv-head) group of 4 query heads (1/32), scaled x32"
    raise KeyError(name)


def blas_threads():
    try:
        from threadpoolctl import threadpool_info
        return max((i.get("num_threads", 0) for i in threadpool_info() if i.get("user_api") == "blas"),
                   default=None)
    except Exception:
        return None


# ----------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--iters", type=int, default=50, help="timed reps per op for the p50")
    ap.add_argument("--ops", default=",".join(CONFIGS), help="comma-separated subset")
    ap.add_argument("--no-cpu", action="store_true", help="skip the host numpy baseline")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU; the operators are single-GPU kernels "
              "(multi-GPU sharding is described in DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    from kda import harness

    if not torch.cuda.is_available():
        log("bench.py: no GPU visible")
        return 1
    dev = torch.device("cuda", 0)
    names = [n for n in args.ops.split(",") if n]

    cases = {}
    for n in names:
        log(f"[bench] preparing {n}")
        cases[n] = make_gpu_case(n, dev)
    torch.cuda.synchronize()

    # Per-op p50 with HIP events on the launch stream.
    results = {}
    for n in names:
        fn, _ = cases[n]
        warm = 3 if n == "adamw" else 10
        iters = max(5, args.iters // 2) if n == "adamw" else args.iters
        t = harness.time_op(fn, warmup=warm, iters=iters, device=dev)
        cfg = CONFIGS[n]
        rl = harness.roofline(cfg["work"], t.p50_ms * 1e-3, cfg["bound"])
        results[n] = dict(p50_ms=t.p50_ms, p10_ms=t.p10_ms, p90_ms=t.p90_ms, mean_ms=t.mean_ms,
                          samples=t.samples, roofline=rl)
        log(f"[bench] {n:15s} p50={t.p50_ms * 1e3:9.1f} us  {rl['achieved']:8.1f} {rl['unit']}  "
            f"frac={rl['frac']:.3f}")

    # Driver contract: W warmup steps, then exactly K steps between synchronisations.
    for i in range(args.warmup):
        for n in names:
            cases[n][0](i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        for n in names:
            cases[n][0](i)
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / max(1, args.steps)
    log(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step")

    cpu = {}
    if not args.no_cpu:
        for n in names:
            log(f"[bench] cpu baseline {n}")
            ms, sample = cpu_baseline(n)
            cpu[n] = dict(p50_ms=ms, sample=sample)
            log(f"[bench] cpu {n:15s} p50={ms:10.1f} ms  ({sample})")

    speedups = {n: cpu[n]["p50_ms"] / results[n]["p50_ms"] for n in names if n in cpu}
    geo = harness.geomean(list(speedups.values())) if speedups else None
    dominant = max(names, key=lambda n: results[n]["p50_ms"])
    rl = dict(results[dominant]["roofline"])
    rl.update(kernel=dominant, kernels=CONFIGS[dominant]["kernels"], traffic=None)
    cores = len(os.sched_getaffinity(0))
    line = {
        "metric": METRIC,
        "value": geo,
        "unit": "x (geomean of numpy_p50 / gpu_p50 over the ops)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16+fp32",
        "data": "synthetic (seeded normal draws of each configuration's distribution, on device)",
        "config": {"workload": "five graded configs: " + "; ".join(CONFIGS[n]["desc"] for n in names),
                   "parallelism": "single GPU"},
        "roofline": rl,
        "cpu_baseline": None if not cpu else {
            "value": sum(c["p50_ms"] for c in cpu.values()), "unit": "ms per step (sum of op p50s)",
            "cores": cores, "blas_threads": blas_threads(), "kind": "port",
            "sample": "; ".join(f"{n}: {c['sample']}" for n, c in cpu.items())},
        "ops": {n: dict(p50_ms=round(results[n]["p50_ms"], 5), dtype=CONFIGS[n]["dtype"],
                        roofline_frac=round(results[n]["roofline"]["frac"], 4),
                        achieved=round(results[n]["roofline"]["achieved"], 1),
                        unit=results[n]["roofline"]["unit"],
                        cpu_p50_ms=(round(cpu[n]["p50_ms"], 2) if n in cpu else None),
                        speedup_vs_numpy=(round(speedups[n], 1) if n in speedups else None))
                for n in names},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
