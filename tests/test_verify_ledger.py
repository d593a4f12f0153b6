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
    with pytest.raises(verify.CaseError, match="lists no operator 'bmm'"):
        verify.resolve_case(CASES, "bmm")
    with pytest.raises(verify.CaseError, match="case '7' is not listed"):
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


def test_build_baselines_writes_reference_format(tmp_path, capsys):
    """--build-baselines runs on the host alone (no GPU): each case's numpy forward,
    timed, written as {"op[case=id]": {baseline_latency_ms, case_id, kernel, op}}
    (the reference's baselines.json format), merged into an existing file, and read
    back as the speedup denominator."""
    path = tmp_path / "baselines.json"
    path.write_text(json.dumps({"other[case=0]": {"baseline_latency_ms": 9.0, "case_id": "0",
                                                  "kernel": "k.py", "op": "other"}}))
    rc = verify.main(["--nkibench-root", str(CASES), "--build-baselines", "--baselines", str(path)])
    out = capsys.readouterr().out
    assert rc == 0 and out.count("BASELINE ") == 3 and "3 baselines written" in out
    data = json.loads(path.read_text())
    assert set(data) == {"other[case=0]", "silu[case=1]", "matmul[case=1]", "add_rmsnorm_matmul[case=1]"}
    ent = data["matmul[case=1]"]
    assert set(ent) == {"baseline_latency_ms", "case_id", "kernel", "op"}
    assert ent["case_id"] == "1" and ent["op"] == "matmul" and ent["baseline_latency_ms"] > 0
    assert ent["kernel"].startswith("matmul_small.py::forward (host numpy")
    c = verify.resolve_case(CASES, "matmul")
    assert verify.baseline_from_file(data, c) == ent["baseline_latency_ms"]


class _Shape:
    def __init__(self, *shape):
        self.shape = shape


def test_roofline_work_matches_the_bench_tables():
    """kda.roofline's work per call, from forward() shapes, equals bench.py's
    NKIBench table (work, bound, fp32-equivalent flops) at every NKIBench shape."""
    import bench
    from kda import roofline
    for op, cfg in bench.NKIBENCH.items():
        names = verify.OPS[op][1]
        shapes = bench._nki_shapes(op, cfg["dims"])
        arrays = [n for n in names if n != "eps"]
        assert len(arrays) == len(shapes), op
        inputs = {n: _Shape(*sh) for n, sh in zip(arrays, shapes)}
        w = roofline.op_work(op, inputs)
        assert w.bound == cfg["bound"] and w.work == cfg["work"], op
        if "useful" in cfg:
            assert w.useful_flops == cfg["useful"], op


def test_roofline_metrics_and_digest():
    from kda import roofline
    m = roofline.metrics("silu", {"x": _Shape(2048, 8192)}, 24e-6)
    assert m["bound"] == "hbm" and m["unit"] == "GB/s"
    assert math.isclose(m["achieved"], 2048 * 8192 * 8 / 24e-6 / 1e9)
    assert math.isclose(m["roofline_frac"], 2048 * 8192 * 8 / 24e-6 / 8e12)
    assert roofline.digest(m) == "HBM 5.59 TB/s = 0.70 of 8 TB/s; HBM algorithmic 134.2MB"
    m = roofline.metrics("matmul", {"lhs": _Shape(4096, 5120), "rhs": _Shape(5120, 12288)}, 1.25e-3,
                         {"read_bytes": 512.0e6, "write_bytes": 201.3e6})
    f = 2 * 4096 * 5120 * 12288
    assert math.isclose(m["roofline_frac"], 3 * f / 1.25e-3 / 2.5e15)
    assert math.isclose(m["fp32_tflops"], f / 1.25e-3 / 1e12)
    d = roofline.digest(m)
    assert d.startswith("MFMA 1237 TFLOP/s issued = 0.49 of 2.5 PFLOP/s; fp32-equivalent 412 TFLOP/s")
    assert "HBMrd=512.0MB HBMwr=201.3MB" in d
    tiny = roofline.metrics("matmul", {"lhs": _Shape(128, 256), "rhs": _Shape(256, 192)}, 22.5e-6)
    assert roofline.digest(tiny).startswith("MFMA 1.68 TFLOP/s issued = 0.000671 of 2.5 PFLOP/s")
    with pytest.raises(KeyError):
        roofline.op_work("conv", {})


def test_traffic_applies_only_at_its_shapes(tmp_path):
    c = verify.load_case_module(CASES / "silu_small.py", "silu")
    prof = tmp_path / "traffic.md"
    prof.write_text("# profile\n\n```json\n" + json.dumps(
        {"silu": {"read_bytes": 256000, "write_bytes": 256000, "shapes": {"x": [64, 1000]}}}) + "\n```\n")
    t = verify.load_traffic(prof)
    inputs = c.draw(0)
    assert verify.traffic_for(t, c, inputs)["read_bytes"] == 256000
    assert verify.traffic_for(t, c, {"x": np.zeros((64, 999), np.float32)}) is None
    assert verify.traffic_for(None, c, inputs) is None


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
    assert out.count("  digest: ") == 3
    assert "  digest: MFMA " in out and "  digest: HBM " in out
    s = ledger.summarize(tmp_path)
    assert s["n_with_validated"] == 3
    rec = json.loads((tmp_path / "matmul" / "candidates.jsonl").read_text().splitlines()[0])
    assert rec["metrics"]["bound"] == "mfma" and 0 < rec["metrics"]["roofline_frac"] < 1
    assert "digest: MFMA" in rec["notes"]


@pytest.mark.gpu
def test_verify_positional_mapping_and_fast(tmp_path, capsys):
    rc = verify.main(["--op", "silu", "--case-module", str(CASES / "silu_renamed.py"), "--fast", "--json"])
    res = json.loads(capsys.readouterr().out)
    assert rc == 0 and res[0]["passed"] and res[0]["seeds"] == [42]
