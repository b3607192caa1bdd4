"""The request-level harness on the CPU: its summary and A/A verdict, the orchestrator's files and order, and one
worker cell on a tiny random-init model (the HFFN arm on a dense stand-in runtime, so that the gates and windows run
without a GPU). The criteria are those of ``runtime/common/pythia/hffn_pythia/bench_request.py:172-196``."""
from __future__ import annotations

import json

import pytest

from hffn_amd import bench_request, pythia
from tests.test_pythia import TINY, DenseStandIn


def _row(size, density, shape, dense, hffn, copy):
    return {"size": size, "density": density, "shape": shape, "samples_ms": {"dense": [dense], "hffn": [hffn], "hffn_copy": [copy]}}


def test_summary_and_verdict():
    rows = [_row(70, 20, "decode_b1", 10.0, 9.0, 9.1), _row(70, 20, "decode_b1", 10.2, 9.2, 9.2), _row(70, 20, "prefill_b1", 4.0, 5.0, 5.05)]
    cells = bench_request.summarize(rows)
    decode = next(c for c in cells if c["shape"] == "decode_b1")
    assert decode["sessions"] == 2 and decode["ms"]["dense"] == pytest.approx(10.1)
    assert decode["hffn_over_dense"] == pytest.approx((0.9 + 9.2 / 10.2) / 2)
    judged = bench_request.verdict(cells, complete=True, gate_passed=True)
    assert judged["admissible"] and judged["aa_values"] == 3
    shaky = bench_request.summarize(rows + [_row(70, 20, "prefill_b4", 4.0, 5.0, 5.5)])
    assert not bench_request.verdict(shaky, complete=True, gate_passed=True)["admissible"]  # 3/4 A/A within 3 %
    assert not bench_request.verdict(cells, complete=True, gate_passed=False)["admissible"]
    assert bench_request.verdict(cells, complete=False, gate_passed=True) == {"admissible": False, "reason": "incomplete coverage"}


def _cpu_adapter():
    load = lambda model_dir, export_dir, ffn, device: pythia.load_pythia(model_dir, export_dir, ffn, "cpu",  # noqa: E731
                                                                         make_runtime=DenseStandIn)
    return bench_request.Adapter(name="CPU stand-in", load_pythia=load, device="cpu", synchronize=lambda: None,
                                 state=lambda: {"device": "cpu"}, versions=lambda: "test", describe=lambda model: {})


def test_orchestrator_files_and_order(tmp_path):
    jobs = []

    def run_cell(job):
        jobs.append(job)
        row = {**{k: v for k, v in job.items() if k != "assets"}, "samples_ms": {a: [1.0, 1.0] for a in bench_request.ARMS},
               "repeats": 3, "gate_passed": True}
        return 0, "log line\n" + json.dumps(row) + "\n", ""

    code = bench_request.orchestrate(_cpu_adapter(), "smoke", tmp_path / "assets", tmp_path / "out", sessions=2, run_cell=run_cell)
    assert code == 0
    assert [(j["session"], j["shape"]) for j in jobs] == [(0, "prefill_b1"), (0, "decode_b1"), (1, "decode_b1"), (1, "prefill_b1")]
    assert [j["parity"] for j in jobs] == [0, 1, 0, 1]
    for name in ("config.json", "provenance.json", "manifest.json", "raw.jsonl", "summary.json", "REPORT.md"):
        assert (tmp_path / "out" / name).exists(), name
    summary = json.loads((tmp_path / "out" / "summary.json").read_text())
    assert summary["verdict"]["admissible"] and len(summary["cells"]) == 2
    assert json.loads((tmp_path / "out" / "manifest.json").read_text())["status"] == "passed"


def test_orchestrator_stops_on_a_failed_gate(tmp_path):
    def run_cell(job):
        row = {**{k: v for k, v in job.items() if k != "assets"}, "samples_ms": {a: [] for a in bench_request.ARMS}, "repeats": None,
               "gate_passed": False}
        return 4, json.dumps(row), ""

    assert bench_request.orchestrate(_cpu_adapter(), "smoke", tmp_path, tmp_path / "out", run_cell=run_cell) == 1
    summary = json.loads((tmp_path / "out" / "summary.json").read_text())
    assert summary["failure"]["returncode"] == 4 and summary["verdict"] is None


def test_worker_cell_on_a_tiny_model(tmp_path):
    assert bench_request.prepare(tmp_path, {1: TINY}, [50])
    assert bench_request.prepare(tmp_path, {1: TINY}, [50]) == []  # nothing missing the second time
    cell = {"size": 1, "density": 50, "shape": "decode_b1", "session": 0, "parity": 1, "blocks": 1, "window_ms": 1.0,
            "assets": str(tmp_path)}
    row = bench_request.worker(_cpu_adapter(), cell)
    assert row["gate_passed"] and row["bitwise_copy"] and row["hffn_vs_dense_relative_gap"] <= bench_request.GUARD
    assert all(len(row["samples_ms"][arm]) == 2 and min(row["samples_ms"][arm]) > 0 for arm in bench_request.ARMS)  # both orders
    assert "assets" not in row
