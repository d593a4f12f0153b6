"""kda.verify (NKIBench case-module loader + scoring contract) and kda.ledger
(benchmark.csv / candidates.jsonl in the reference's format, summary geomean).

CPU tests drive the loader, seeding, name mapping, the relative-L2 gate and the
ledger with a host stand-in for the GPU call; the GPU tests run the CLI end to end."""
import csv
import json
import math
from pathlib import Path

import numpy as np
import pytest

from kda import ledger, verify

CASES = Path(__file__).resolve().parent / "cases"


def test_case_module_loads_and_maps_forward_names():
    c = verify.load_case_module(CASES / "add_rmsnorm_matmul_small.py", "add_rmsnorm_matmul")
    assert c.param_names == ["x", "w", "eps", "z", "g"]
    assert c.rel_tol == 2e-5
    d = c.draw(0)
    assert list(d) == ["x", "w", "eps", "z", "g"]
    assert d["eps"] == 1e-5 and d["x"].shape == (96, 128)
    assert verify.load_case_module(CASES / "silu_small.py", "mamba").rel_tol == 3e-5


def test_seeds_draw_distinct_but_reproducible_inputs():
    c = verify.load_case_module(CASES / "silu_small.py", "silu")
    a0, a0b, a21 = c.draw(0)["x"], c.draw(0)["x"], c.draw(21)["x"]
    np.testing.assert_array_equal(a0, a0b)
    assert not np.array_equal(a0, a21)
    np.random.seed(0)
    np.testing.assert_array_equal(a0, np.random.normal(0.0, 1.0, (64, 1000)).astype(np.float32))


def test_resolve_case_through_summary_json():
    c = verify.resolve_case(CASES, "matmul")
    assert c.case_id == "1" and c.module_path.name == "matmul_small.py"
    with pytest.raises(verify.CaseError, match="not in summary.json"):
        verify.resolve_case(CASES, "bmm")
    with pytest.raises(verify.CaseError, match="no case"):
        verify.resolve_case(CASES, "matmul", "7")


def test_missing_module_and_missing_functions(tmp_path):
    with pytest.raises(verify.CaseError, match="does not exist"):
        verify.load_case_module(tmp_path / "nope.py", "silu")
    bad = tmp_path / "bad.py"
    bad.write_text("def get_inputs():\n    return []\n")
    with pytest.raises(verify.CaseError, match="forward"):
        verify.load_case_module(bad, "silu")


def test_cli_without_a_golden_exits_2(monkeypatch, capsys):
    monkeypatch.delenv("NKIBENCH_ROOT", raising=False)
    assert verify.main(["--op", "silu"]) == 2
    assert "no golden" in capsys.readouterr().err
    assert verify.main(["--case-module", str(CASES / "silu_small.py")]) == 2


def _host_call(op, case, inputs, device):
    """Stand-in for the GPU call: the case's own forward, optionally perturbed."""
    out = case.forward(**inputs)
    return lambda: out * np.float32(1.0 + _host_call.rel)


def test_gate_passes_and_fails_on_relative_l2(monkeypatch):
    monkeypatch.setattr(verify, "make_call", _host_call)
    c = verify.load_case_module(CASES / "silu_small.py", "silu")
    _host_call.rel = 1e-6
    r = verify.score_case(c, verify.SEEDS, None, time_it=False)
    assert r.passed and sorted(r.rel_l2) == verify.SEEDS
    assert all(abs(e - 1e-6) < 1e-7 for e in r.rel_l2.values())
    _host_call.rel = 3e-5                       # over the 2e-5 gate
    r = verify.score_case(c, verify.SEEDS, None, time_it=False)
    assert not r.passed and "rel-L2 over 2e-05" in r.error
    assert verify.line(r).startswith("FAIL silu[case=0]")


def test_rel_l2_definition():
    want = np.array([3.0, 4.0], dtype=np.float32)
    assert verify.rel_l2(want, want) == 0.0
    assert math.isclose(verify.rel_l2(np.array([3.0, 5.0]), want), 1.0 / 5.0)
    with pytest.raises(verify.CaseError):
        verify.rel_l2(np.zeros(3), want)


def test_baseline_lookup_in_reference_format():
    c = verify.resolve_case(CASES, "silu")
    base = {"silu[case=1]": {"baseline_latency_ms": 1.0224, "case_id": "1"}}
    assert verify.baseline_from_file(base, c) == 1.0224
    assert verify.baseline_from_file({"matmul": {"baseline_latency_ms": 2.0}}, c) is None


def test_ledger_rows_and_summary(tmp_path):
    full = verify.SEEDS
    recs = [
        ledger.record("silu", "libkda v1", "", True, 0.024, 120.0, full, "scored"),
        ledger.record("silu", "libkda v2", "libkda v1", True, 0.020, 150.0, full, "scored"),
        ledger.record("silu", "screen", "", True, 0.010, 300.0, [42], "fast-screen"),   # not full gate
        ledger.record("silu", "bad", "", False, None, None, full, "scored", notes="rel-L2 over"),
        ledger.record("matmul", "libkda v1", "", True, 1.2, 40.0, full, "scored"),
        ledger.record("matmul", "rej", "", True, 1.0, 99.0, full, "REJECTED"),
    ]
    for r in recs:
        ledger.append(tmp_path, r)
    with (tmp_path / "silu" / "benchmark.csv").open(newline="") as f:
        rows = list(csv.reader(f))
    assert rows[0] == ledger.CSV_HEADER
    assert rows[0] == "timestamp,op,candidate,parent,passed,latency_ms,speedup,notes".split(",")
    assert len(rows) == 5 and rows[2][4] == "true" and rows[4][4] == "false" and rows[4][5] == ""
    lines = (tmp_path / "silu" / "candidates.jsonl").read_text().splitlines()
    assert json.loads(lines[0])["seeds"] == full
    s = ledger.summarize(tmp_path)
    by_op = {r["op"]: r for r in s["ops"]}
    assert by_op["silu"]["best_speedup"] == 150.0 and by_op["silu"]["n_validated"] == 2
    assert by_op["matmul"]["best_speedup"] == 40.0
    assert math.isclose(s["geomean_best_speedup"], math.sqrt(150.0 * 40.0))
    assert ledger.main([str(tmp_path), "--json"]) == 0


@pytest.mark.gpu
def test_verify_cli_end_to_end(tmp_path, capsys):
    rc = verify.main(["--nkibench-root", str(CASES), "--iters", "20", "--ledger", str(tmp_path)])
    out = capsys.readouterr().out
    print(out)
    assert rc == 0
    assert out.count("PASS ") == 3 and "geomean speedup" in out
    s = ledger.summarize(tmp_path)
    assert s["n_with_validated"] == 3


@pytest.mark.gpu
def test_verify_positional_mapping_and_fast(tmp_path, capsys):
    rc = verify.main(["--op", "silu", "--case-module", str(CASES / "silu_renamed.py"), "--fast", "--json"])
    res = json.loads(capsys.readouterr().out)
    assert rc == 0 and res[0]["passed"] and res[0]["seeds"] == [42]
