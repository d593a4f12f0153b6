"""Evidence ledger in the reference's per-operator format.

Each operator directory ``<root>/<op>/`` holds

* ``benchmark.csv`` with the header
  ``timestamp,op,candidate,parent,passed,latency_ms,speedup,notes``
  (the schema created by scripts/new-task.sh:33), one row per scored run;
* ``candidates.jsonl``, one JSON record per run with the keys the reference's
  records use most (``id, op, candidate, parent, timestamp, passed, verdict,
  seeds, latency_ms, baseline_latency_ms, speedup, metrics, notes``;
  e.g. workspaces/silu/candidates.jsonl:1).

``summarize`` follows scripts/summary.py:29-95,137-141: a record counts only if
it passed the full five-seed gate with a numeric speedup and its verdict is not
a rejection, a drop or a fast screen; per operator the best such speedup is
reported, and the aggregate is their geometric mean.  Beside it, the latest
passing record of each operator (bench.py rows are checked on one seed) and the
geomean of those are reported.

    python -m kda.ledger <root> [--json]
"""
from __future__ import annotations

import argparse
import csv
import json
import math
import os
import sys
import time
from pathlib import Path
from typing import Any, Dict, Iterable, List, Optional

CSV_HEADER = ["timestamp", "op", "candidate", "parent", "passed", "latency_ms", "speedup", "notes"]
FULL_GATE_SEEDS = frozenset({0, 21, 42, 63, 84})
_NON_VALIDATED_VERDICTS = ("REJECT", "DROPPED", "SCREEN")


def utc_timestamp(t: Optional[float] = None) -> str:
    return time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime(time.time() if t is None else t))


def record(op: str, candidate: str, parent: str, passed: bool, latency_ms: Optional[float],
           speedup: Optional[float], seeds: Iterable[int], verdict: str, notes: str = "",
           baseline_latency_ms: Optional[float] = None, metrics: Optional[Dict[str, Any]] = None,
           **extra: Any) -> Dict[str, Any]:
    """One ledger record (the candidates.jsonl shape)."""
    ts = utc_timestamp()
    rec: Dict[str, Any] = {
        "id": f"{op}@{ts}", "op": op, "candidate": candidate, "parent": parent,
        "timestamp": ts, "passed": bool(passed), "verdict": verdict,
        "seeds": sorted(int(s) for s in seeds),
        "latency_ms": None if latency_ms is None else round(float(latency_ms), 6),
        "baseline_latency_ms": None if baseline_latency_ms is None else round(float(baseline_latency_ms), 6),
        "speedup": None if speedup is None else round(float(speedup), 3),
        "metrics": metrics or {}, "notes": notes,
    }
    rec.update(extra)
    return rec


def append(root: os.PathLike, rec: Dict[str, Any]) -> Path:
    """Appends `rec` to <root>/<op>/benchmark.csv (header written on creation) and
    to <root>/<op>/candidates.jsonl; returns the operator directory."""
    ws = Path(root) / rec["op"]
    ws.mkdir(parents=True, exist_ok=True)
    path = ws / "benchmark.csv"
    new = not path.exists() or path.stat().st_size == 0
    with path.open("a", newline="") as f:
        w = csv.writer(f)
        if new:
            w.writerow(CSV_HEADER)
        w.writerow([rec["timestamp"], rec["op"], rec["candidate"], rec["parent"],
                    "true" if rec["passed"] else "false",
                    "" if rec["latency_ms"] is None else f"{rec['latency_ms']:.6g}",
                    "" if rec["speedup"] is None else f"{rec['speedup']:.6g}",
                    rec.get("notes", "")])
    with (ws / "candidates.jsonl").open("a") as f:
        f.write(json.dumps(rec, sort_keys=False) + "\n")
    return ws


def read_csv(root: os.PathLike, op: str) -> List[Dict[str, str]]:
    path = Path(root) / op / "benchmark.csv"
    if not path.exists():
        return []
    with path.open(newline="") as f:
        rows = list(csv.DictReader(f))
    return rows


def is_validated(d: Dict[str, Any]) -> bool:
    """Passed the full five-seed gate with a numeric speedup, and the verdict is not
    a rejection, drop or screen (scripts/summary.py:33-42)."""
    if not d.get("passed") or not isinstance(d.get("speedup"), (int, float)):
        return False
    seeds = d.get("seeds")
    if not (isinstance(seeds, (list, tuple)) and FULL_GATE_SEEDS.issubset(set(seeds))):
        return False
    v = str(d.get("verdict", "")).upper()
    return not any(bad in v for bad in _NON_VALIDATED_VERDICTS)


def scan_op(root: os.PathLike, op: str) -> Dict[str, Any]:
    """Best validated speedup of one operator, the count of validated records, and
    the latest passing record of any kind (e.g. a bench row checked on one seed)."""
    best = None
    latest = None
    n_pass = n_all = 0
    path = Path(root) / op / "candidates.jsonl"
    if path.exists():
        for line in path.read_text().splitlines():
            line = line.strip()
            if not line:
                continue
            try:
                d = json.loads(line)
            except json.JSONDecodeError:
                continue
            n_all += 1
            if d.get("passed") and isinstance(d.get("speedup"), (int, float)):
                latest = d
            if is_validated(d):
                n_pass += 1
                if best is None or d["speedup"] > best["speedup"]:
                    best = d
    return {"op": op, "best_speedup": best["speedup"] if best else None,
            "best_candidate": best["candidate"] if best else None,
            "best_latency_ms": best["latency_ms"] if best else None,
            "n_validated": n_pass, "n_records": n_all,
            "latest_speedup": latest["speedup"] if latest else None,
            "latest_latency_ms": latest["latency_ms"] if latest else None,
            "latest_seeds": latest["seeds"] if latest else None,
            "latest_verdict": latest.get("verdict") if latest else None}


def summarize(root: os.PathLike) -> Dict[str, Any]:
    root = Path(root)
    ops = sorted(p.name for p in root.iterdir() if p.is_dir()) if root.is_dir() else []
    rows = [scan_op(root, op) for op in ops]
    speeds = [r["best_speedup"] for r in rows if r["best_speedup"]]
    geo = math.exp(sum(math.log(s) for s in speeds) / len(speeds)) if speeds else None
    lat = [r["latest_speedup"] for r in rows if r["latest_speedup"]]
    geo_latest = math.exp(sum(math.log(s) for s in lat) / len(lat)) if lat else None
    return {"ops": rows, "n_with_validated": len(speeds), "n_ops": len(rows),
            "geomean_best_speedup": geo,
            "range": [min(speeds), max(speeds)] if speeds else None,
            "n_with_latest": len(lat), "geomean_latest_speedup": geo_latest}


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(description="Summarise an evidence ledger directory.")
    ap.add_argument("root", help="ledger root: one sub-directory per operator")
    ap.add_argument("--json", action="store_true", help="machine-readable output")
    args = ap.parse_args(argv)
    s = summarize(args.root)
    if args.json:
        print(json.dumps(s, indent=2))
        return 0
    rows = sorted(s["ops"], key=lambda r: r["best_speedup"] or r["latest_speedup"] or -1, reverse=True)
    print(f"{'op':26s} {'best (5 seeds)':>15s} {'p50 ms':>10s}  {'latest':>12s} {'p50 ms':>10s}  "
          f"validated/records")
    print("-" * 96)
    for r in rows:
        bs = f"{r['best_speedup']:.3f}x" if r["best_speedup"] else "-"
        lat = f"{r['best_latency_ms']:.4f}" if r["best_latency_ms"] is not None else "-"
        ls = f"{r['latest_speedup']:.3f}x" if r["latest_speedup"] else "-"
        llat = f"{r['latest_latency_ms']:.4f}" if r["latest_latency_ms"] is not None else "-"
        print(f"{r['op']:26s} {bs:>15s} {lat:>10s}  {ls:>12s} {llat:>10s}  "
              f"{r['n_validated']}/{r['n_records']}")
    print("-" * 96)
    if s["geomean_latest_speedup"]:
        print(f"geomean(latest passing)     : {s['geomean_latest_speedup']:.3f}x over "
              f"{s['n_with_latest']} ops (latest rows may be single-seed bench checks)")
    if s["geomean_best_speedup"]:
        lo, hi = s["range"]
        print(f"ops with a validated result : {s['n_with_validated']}/{s['n_ops']}")
        print(f"geomean(best speedup)       : {s['geomean_best_speedup']:.3f}x   "
              f"(range {lo:.3f}x .. {hi:.3f}x)")
    else:
        print("no validated results yet")
    return 0


if __name__ == "__main__":
    sys.exit(main())
