"""verify.py-style scoring of the library's operators against NKIBench case modules.

    python -m kda.verify --op silu --case-module PATH [--fast] [--seeds 0,21,...]
    python -m kda.verify --op matmul --nkibench-root DIR [--case-id ID]
    python -m kda.verify --pilot | (no selector: every op of summary.json) --nkibench-root DIR
    python -m kda.verify --build-baselines [--baselines baselines.json] <case selection>
    options: --baselines baselines.json  --traffic FILE  --ledger DIR  --json  --iters N
             --warmup N  --rtol X

Follows the reference's evaluation contract (verify.py:13-65):
- The golden is the case module's own numpy ``forward(...)``.  A case module is
  an NKIBench reference file: ``get_inputs()`` returns the natural-layout inputs
  and ``forward(*inputs)`` the golden output.  Inputs are keyed by forward()'s
  parameter names (adapter/nkibench_case.py:147-155,199-216).  With
  ``--nkibench-root`` (or $NKIBENCH_ROOT) the module is found through
  ``summary.json`` the way adapter/nkibench_case.py:235-264 resolves a case.
- Each seed of [0, 21, 42, 63, 84] runs ``np.random.seed(seed)`` before
  ``get_inputs()``.  Unlike adapter/nkibench_case.py:45-50, which reseeds 42
  for every seed, each seed here draws different inputs.  ``--fast`` uses seed
  42 only, as the reference's fast screen does.
- passed = every seed satisfies ||out - golden||_2 < rtol * ||golden||_2, with
  norms in float64.  rtol is 2e-5, or 3e-5 for mamba
  (adapter/nkibench_case.py:51-53).
- latency_ms = p50 of HIP-event timings on the launch stream, after warm-up.
- speedup = baseline_latency_ms / latency_ms.  The baseline is the entry in
  ``--baselines`` (the reference's baselines.json format) when one is given.
  Otherwise it is the case's numpy forward timed on this host, p50 of 3 after
  one warm-up.
- ``--build-baselines`` measures each case's baseline (its numpy forward on this
  host, p50 of 3 after one warm-up) and writes ``{"op[case=id]": {baseline_latency_ms,
  case_id, kernel, op}}`` into the ``--baselines`` file (default baselines.json),
  the format later runs read as their speedup denominator (verify.py:23,57-59).
- ``summary_metrics`` holds the p10/p90 latency, the operator's bound (HBM or
  MFMA), its achieved rate and fraction of the MI355X peak at the p50, and its
  algorithmic HBM bytes (``kda.roofline``); with ``--traffic`` (the measured HBM
  read/write bytes of a rocprofv3 profile at the same shapes) also those bytes.
  Each op's line is followed by a one-line digest of them (verify.py:48-50,
  README.md:146-147), which is also the ledger row's note.
- One PASS/FAIL line per op, then the geomean of the speedups.  The exit code is
  0 only if every scored op passed, or with ``--build-baselines`` every baseline
  was measured (verify.py:52-61).

The library's callable for each op takes the forward() arguments in natural
layout (kda.ops).  Keyword names are used when they match the callable's
parameters; otherwise the inputs are passed in forward() order.
"""
from __future__ import annotations

import argparse
import importlib.util
import inspect
import json
import math
import os
import statistics
import sys
import time
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Any, Callable, Dict, List, Optional, Sequence

import numpy as np

SEEDS: List[int] = [0, 21, 42, 63, 84]
FAST_SEEDS: List[int] = [42]
DEFAULT_REL_TOL = 2e-5
REL_TOL_OVERRIDES = {"mamba": 3e-5}
PILOT_OPS = ["matmul", "silu", "rmsnorm_matmul"]

# op -> name of the kda.ops callable and its parameters in forward() order.
OPS: Dict[str, tuple] = {
    "silu": ("silu", ("x",)),
    "adamw": ("adamw", ("theta", "g", "m", "v")),
    "rope_single_freq_apply": ("rope_single_freq_apply", ("x_in", "cos", "sin")),
    "mamba": ("mamba", ("delta", "u", "a", "b", "c")),
    "matmul": ("matmul", ("lhs", "rhs")),
    "transpose_matmul": ("transpose_matmul", ("lhs", "rhs")),
    "bmm": ("bmm", ("lhs", "rhs")),
    "bmm_softmax": ("bmm_softmax", ("lhs", "rhs")),
    "lora": ("lora", ("x", "w", "a", "b")),
    "rmsnorm_matmul": ("rmsnorm_matmul", ("x", "w")),
    "add_rmsnorm_matmul": ("add_rmsnorm_matmul", ("x", "w", "eps", "z", "g")),
    "matmul_add_rmsnorm": ("matmul_add_rmsnorm", ("x", "w", "eps", "z", "g")),
    "swiglu": ("swiglu", ("x", "w_up", "w_down", "w_gate")),
    "gqa_full": ("gqa_full", ("q", "k", "v")),
}


class CaseError(ValueError):
    """A case module or summary.json entry that cannot be used."""


# ----------------------------------------------------------------- case modules

@dataclass
class Case:
    op: str
    case_id: str
    module_path: Path
    get_inputs: Callable[[], Any]
    forward: Callable[..., Any]
    param_names: List[str]
    rel_tol: float

    @property
    def name(self) -> str:
        return f"{self.op}[case={self.case_id}]"

    def draw(self, seed: int) -> Dict[str, Any]:
        """Natural-layout inputs keyed by forward()'s parameter names."""
        np.random.seed(seed)
        vals = self.get_inputs()
        if isinstance(vals, dict):
            return dict(vals)
        vals = list(vals)
        if len(vals) != len(self.param_names):
            raise CaseError(f"{self.name}: get_inputs() returned {len(vals)} values for "
                            f"forward{tuple(self.param_names)}")
        return {n: v for n, v in zip(self.param_names, vals)}


def forward_param_names(fn: Callable[..., Any]) -> List[str]:
    """Positional parameter names of forward() (adapter/nkibench_case.py:199-216)."""
    names = [p.name for p in inspect.signature(fn).parameters.values()
             if p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD) and p.name != "self"]
    if not names:
        raise CaseError("forward() has no positional parameters")
    return names


def load_case_module(path: os.PathLike, op: str, case_id: str = "0",
                     rel_tol: Optional[float] = None) -> Case:
    """Imports an NKIBench reference file and returns its case.  The file is the
    caller's: it is executed, as the reference's profiler executes it."""
    path = Path(path).resolve()
    if not path.is_file():
        raise CaseError(f"case module {path} does not exist")
    spec = importlib.util.spec_from_file_location(f"_kda_case_{op}_{abs(hash(path))}", path)
    if spec is None or spec.loader is None:
        raise CaseError(f"cannot import {path}")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    for attr in ("get_inputs", "forward"):
        if not callable(getattr(mod, attr, None)):
            raise CaseError(f"{path} defines no {attr}()")
    return Case(op=op, case_id=str(case_id), module_path=path, get_inputs=mod.get_inputs,
                forward=mod.forward, param_names=forward_param_names(mod.forward),
                rel_tol=rel_tol if rel_tol is not None else REL_TOL_OVERRIDES.get(op, DEFAULT_REL_TOL))


def load_summary(root: os.PathLike) -> Dict[str, Any]:
    path = Path(root) / "summary.json"
    try:
        return json.loads(path.read_text())
    except OSError as e:
        raise CaseError(f"cannot read {path}: {e}") from e


def resolve_case(root: os.PathLike, op: str, case_id: Optional[str] = None,
                 rel_tol: Optional[float] = None) -> Case:
    """summary.json[op]["cases"][case_id]["impls"][0]["task"] is the reference file
    (adapter/nkibench_case.py:235-264); a single case is the default."""
    summary = load_summary(root)
    if op not in summary:
        raise CaseError(f"summary.json lists no operator {op!r} (it lists {', '.join(sorted(summary))})")
    cases = summary[op]["cases"]
    if case_id is None:
        if len(cases) != 1:
            raise CaseError(f"{op} lists {len(cases)} cases ({', '.join(sorted(cases))}): choose one with --case-id")
        case_id = next(iter(cases))
    if case_id not in cases:
        raise CaseError(f"{op}: case {case_id!r} is not listed (listed: {', '.join(sorted(cases))})")
    task = cases[case_id]["impls"][0]["task"]
    return load_case_module(Path(root) / task, op, case_id, rel_tol)


# ----------------------------------------------------------------- scoring

@dataclass
class Result:
    """Per-operator result in the shape of the reference's verify.py output."""
    op: str
    case: str
    passed: bool
    latency_ms: Optional[float]
    error: Optional[str] = None
    seeds: List[int] = field(default_factory=list)
    rel_l2: Dict[int, float] = field(default_factory=dict)
    rel_tol: float = DEFAULT_REL_TOL
    baseline_latency_ms: Optional[float] = None
    baseline_kind: Optional[str] = None
    speedup: Optional[float] = None
    summary_metrics: Dict[str, Any] = field(default_factory=dict)


def rel_l2(got: Any, want: Any) -> float:
    """||got - want||_2 / ||want||_2 over the flattened arrays, in float64."""
    g = np.asarray(got, dtype=np.float64).ravel()
    w = np.asarray(want, dtype=np.float64).ravel()
    if g.shape != w.shape:
        raise CaseError(f"output has {g.size} elements, golden {w.size}")
    den = float(np.linalg.norm(w))
    num = float(np.linalg.norm(g - w))
    if den == 0.0:
        return 0.0 if num == 0.0 else math.inf
    return num / den


def _device_args(inputs: Dict[str, Any], device) -> List[Any]:
    """forward()-ordered inputs moved to the device (float arrays as fp32 tensors)."""
    import torch

    def move(v):
        if isinstance(v, np.ndarray):
            if v.dtype.kind == "f":
                return torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)).to(device)
            return torch.from_numpy(np.ascontiguousarray(v)).to(device)
        if isinstance(v, np.generic):
            return v.item()
        return v
    return [move(v) for v in inputs.values()]


def make_call(op: str, case: Case, inputs: Dict[str, Any], device) -> Callable[[], Any]:
    """Returns a no-argument callable that runs the library's op on these inputs."""
    from . import ops
    fname, params = OPS[op]
    fn = getattr(ops, fname)
    args = _device_args(inputs, device)
    if len(args) != len(params):
        raise CaseError(f"{case.name}: forward takes {len(args)} inputs, kda.ops.{fname} {len(params)}")
    if set(inputs) == set(params):
        kwargs = dict(zip(inputs.keys(), args))
        return lambda: fn(**kwargs)
    return lambda: fn(*args)


def _host(t: Any) -> np.ndarray:
    import torch
    if isinstance(t, torch.Tensor):
        return t.detach().to("cpu", torch.float32).numpy()
    return np.asarray(t)


def time_host(fn: Callable[[], Any], reps: int = 3) -> float:
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts) * 1e3


def baseline_from_file(baselines: Dict[str, Any], case: Case) -> Optional[float]:
    for key in (case.name, case.op):
        ent = baselines.get(key)
        if isinstance(ent, dict) and isinstance(ent.get("baseline_latency_ms"), (int, float)):
            return float(ent["baseline_latency_ms"])
    return None


def load_traffic(path: os.PathLike) -> Dict[str, Any]:
    """Measured HBM traffic per operator: a JSON object (or the first ```json block
    of a Markdown profile) mapping an operator name to ``{"read_bytes",
    "write_bytes", "shapes": {forward() name: shape}}``."""
    text = Path(path).read_text()
    if "```json" in text:
        text = text.split("```json", 1)[1].split("```", 1)[0]
    data = json.loads(text)
    if not isinstance(data, dict):
        raise CaseError(f"{path}: expected a JSON object of operators")
    return data


def traffic_for(traffic: Optional[Dict[str, Any]], case: Case, inputs: Dict[str, Any]) -> Optional[Dict[str, Any]]:
    """The profile's figures for this case, only when they were measured at the
    same input shapes."""
    if not traffic:
        return None
    ent = traffic.get(case.name) or traffic.get(case.op)
    if not isinstance(ent, dict) or "read_bytes" not in ent or "write_bytes" not in ent:
        return None
    shapes = {k: list(np.shape(v)) for k, v in inputs.items() if np.ndim(v)}
    want = {k: list(v) for k, v in ent.get("shapes", {}).items()}
    return ent if want == shapes else None


def score_case(case: Case, seeds: Sequence[int], device, warmup: int = 20, iters: int = 100,
               baselines: Optional[Dict[str, Any]] = None, time_it: bool = True,
               traffic: Optional[Dict[str, Any]] = None) -> Result:
    """Correctness on every seed, then p50 latency, roofline metrics and speedup on
    the last seed."""
    from . import harness, roofline
    res = Result(op=case.op, case=case.case_id, passed=False, latency_ms=None,
                 seeds=list(seeds), rel_tol=case.rel_tol)
    call = inputs = None
    try:
        for s in seeds:
            inputs = case.draw(s)
            call = make_call(case.op, case, inputs, device)
            got = _host(call())
            want = np.asarray(case.forward(**inputs))
            res.rel_l2[s] = rel_l2(got, want)
    except Exception as e:   # surfaced as a failed op, like the reference's error field
        res.error = f"{type(e).__name__}: {e}"
        return res
    bad = [s for s, e in res.rel_l2.items() if not (e < case.rel_tol)]
    res.passed = not bad
    if bad:
        res.error = f"rel-L2 over {case.rel_tol:g} on seeds {bad}"
        return res
    if time_it and call is not None:
        t = harness.time_op(lambda i: call(), warmup=warmup, iters=iters, device=device)
        res.latency_ms = t.p50_ms
        res.summary_metrics = {"p10_ms": t.p10_ms, "p90_ms": t.p90_ms, "reps": t.samples}
        # the work model reads the operator's own parameter names; a case module's
        # forward() may name them differently, so map them by position
        named = dict(zip(OPS[case.op][1], inputs.values()))
        res.summary_metrics.update(roofline.metrics(case.op, named, t.p50_ms * 1e-3,
                                                    traffic_for(traffic, case, inputs)))
        base = baseline_from_file(baselines, case) if baselines else None
        if base is not None:
            res.baseline_latency_ms, res.baseline_kind = base, "baselines.json"
        else:
            res.baseline_latency_ms = time_host(lambda: case.forward(**inputs))
            res.baseline_kind = f"host numpy forward ({len(os.sched_getaffinity(0))} cores)"
        res.speedup = res.baseline_latency_ms / res.latency_ms
    return res


def geomean(xs: Sequence[float]) -> Optional[float]:
    xs = [x for x in xs if x and x > 0 and math.isfinite(x)]
    return math.exp(sum(math.log(x) for x in xs) / len(xs)) if xs else None


def line(r: Result) -> str:
    tag = "PASS" if r.passed else "FAIL"
    worst = max(r.rel_l2.values()) if r.rel_l2 else float("nan")
    lat = f"p50={r.latency_ms:.4f} ms" if r.latency_ms is not None else "p50=-"
    sp = f"speedup={r.speedup:.3f}x" if r.speedup is not None else "speedup=-"
    err = f"  error: {r.error}" if r.error else ""
    return (f"{tag} {r.op}[case={r.case}]  {lat}  {sp}  rel_l2_max={worst:.3e} "
            f"(tol {r.rel_tol:g}, seeds {r.seeds}){err}")


def digest_line(r: Result) -> str:
    """The one-line bottleneck digest of an op's summary_metrics (empty if untimed)."""
    from . import roofline
    d = roofline.digest(r.summary_metrics)
    return f"  digest: {d}" if d else ""


def build_baselines(cases: Sequence[Case], path: os.PathLike, seed: int = 42,
                    reps: int = 3) -> Dict[str, Any]:
    """Measures every case's baseline (its numpy forward on this host, p50 of
    `reps` after one warm-up, on the inputs of `seed`) and merges the entries into
    the baselines file in the reference's format (verify.py:23,57-59)."""
    path = Path(path)
    data: Dict[str, Any] = json.loads(path.read_text()) if path.exists() else {}
    cores = len(os.sched_getaffinity(0))
    for c in cases:
        inputs = c.draw(seed)
        ms = time_host(lambda: c.forward(**inputs), reps)
        data[c.name] = {"baseline_latency_ms": ms, "case_id": c.case_id,
                        "kernel": f"{c.module_path.name}::forward (host numpy, {cores} cores)",
                        "op": c.op}
    path.write_text(json.dumps(data, indent=2, sort_keys=True) + "\n")
    return data


# ----------------------------------------------------------------- CLI

def _parse(argv: Optional[List[str]]) -> argparse.Namespace:
    ap = argparse.ArgumentParser(prog="python -m kda.verify", description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    sel = ap.add_mutually_exclusive_group()
    sel.add_argument("--op", choices=sorted(OPS), help="one operator")
    sel.add_argument("--pilot", action="store_true", help=f"the pilot subset {PILOT_OPS}")
    ap.add_argument("--case-module", help="NKIBench reference file for --op (get_inputs/forward)")
    ap.add_argument("--case-id", default=None, help="case id in summary.json")
    ap.add_argument("--nkibench-root", default=os.environ.get("NKIBENCH_ROOT"),
                    help="NKIBench root holding summary.json (default $NKIBENCH_ROOT)")
    ap.add_argument("--seeds", default=None, help="comma-separated seeds (default 0,21,42,63,84)")
    ap.add_argument("--fast", action="store_true", help="seed 42 only, fewer timed reps")
    ap.add_argument("--rtol", type=float, default=None, help="override the relative-L2 gate")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--baselines", default=None, help="baselines.json (speedup denominators)")
    ap.add_argument("--build-baselines", action="store_true",
                    help="measure each case's baseline and write it to --baselines (default baselines.json)")
    ap.add_argument("--traffic", default=None,
                    help="measured HBM bytes per op (JSON, or a Markdown profile with a json block)")
    ap.add_argument("--ledger", default=None, help="append results to <DIR>/<op>/benchmark.csv")
    ap.add_argument("--candidate", default=None, help="candidate name recorded in the ledger")
    ap.add_argument("--parent", default="", help="parent name recorded in the ledger")
    ap.add_argument("--json", action="store_true", help="print results as JSON")
    return ap.parse_args(argv)


def cases_for(args: argparse.Namespace) -> List[Case]:
    if args.case_module:
        if not args.op:
            raise CaseError("--case-module needs --op")
        return [load_case_module(args.case_module, args.op, args.case_id or "0", args.rtol)]
    if not args.nkibench_root:
        raise CaseError("no golden: pass --case-module, --nkibench-root or set NKIBENCH_ROOT")
    if args.op:
        ops = [args.op]
    elif args.pilot:
        ops = list(PILOT_OPS)
    else:
        ops = [op for op in load_summary(args.nkibench_root) if op in OPS]
    return [resolve_case(args.nkibench_root, op, args.case_id, args.rtol) for op in ops]


def main(argv: Optional[List[str]] = None) -> int:
    args = _parse(argv)
    try:
        cases = cases_for(args)
    except CaseError as e:
        print(f"verify: {e}", file=sys.stderr)
        return 2
    seeds = FAST_SEEDS if args.fast else (
        [int(s) for s in args.seeds.split(",")] if args.seeds else SEEDS)
    iters = min(args.iters, 20) if args.fast else args.iters
    if args.build_baselines:
        path = args.baselines or "baselines.json"
        try:
            data = build_baselines(cases, path)
        except Exception as e:
            print(f"verify: baseline measurement failed: {type(e).__name__}: {e}", file=sys.stderr)
            return 1
        for c in cases:
            e = data[c.name]
            print(f"BASELINE {c.name}  {e['baseline_latency_ms']:.4f} ms  ({e['kernel']})")
        print(f"{len(cases)} baselines written to {path}")
        return 0
    baselines = json.loads(Path(args.baselines).read_text()) if args.baselines else None
    try:
        traffic = load_traffic(args.traffic) if args.traffic else None
    except (OSError, ValueError) as e:
        print(f"verify: cannot read --traffic: {e}", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("verify: no GPU visible", file=sys.stderr)
        return 1
    device = torch.device("cuda", 0)
    results = [score_case(c, seeds, device, args.warmup, iters, baselines, traffic=traffic)
               for c in cases]

    if args.ledger:
        from . import _lib, ledger
        cand = args.candidate or f"libkda.so v{_lib.version()}"
        for c, r in zip(cases, results):
            ledger.append(args.ledger, ledger.record(
                op=r.op, candidate=cand, parent=args.parent, passed=r.passed,
                latency_ms=r.latency_ms, speedup=r.speedup, seeds=r.seeds,
                verdict="scored" if not args.fast else "fast-screen",
                notes=(r.error or f"rel_l2_max {max(r.rel_l2.values()):.3e}; "
                       f"baseline {r.baseline_kind}; {digest_line(r).strip()}"),
                baseline_latency_ms=r.baseline_latency_ms,
                metrics=r.summary_metrics, case_id=r.case, case_module=str(c.module_path),
                per_seed_rel_l2={str(k): v for k, v in r.rel_l2.items()}))

    if args.json:
        print(json.dumps([asdict(r) for r in results], indent=2, default=str))
    else:
        for r in results:
            print(line(r))
            if digest_line(r):
                print(digest_line(r))
        g = geomean([r.speedup for r in results if r.passed and r.speedup])
        npass = sum(r.passed for r in results)
        print(f"{npass}/{len(results)} passed; geomean speedup "
              f"{'-' if g is None else f'{g:.3f}x'}")
    return 0 if all(r.passed for r in results) else 1


if __name__ == "__main__":
    sys.exit(main())
