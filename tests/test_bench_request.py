"""The request-level harness on the CPU: aggregation and the A/A admissibility rule, the campaign's run order and
files, and one cell on a tiny random-init model (the HFFN arm on a dense stand-in runtime, so that gates and windows
run without a GPU). Criteria: ``runtime/common/pythia/hffn_pythia/bench_request.py:1-20,172-196``."""
from __future__ import annotations

import json

import pytest

from hffn_amd import bench_request, pythia
from tests.test_pythia import TINY, DenseStandIn


def _row(size, density, shape, dense, hffn, copy):
    return {"size": size, "density": density, "shape": shape, "samples_ms": {"dense": [dense], "hffn": [hffn], "hffn_copy": [copy]}}


def test_aggregate_and_admissibility():
    rows = [_row(70, 20, "decode_b1", 10.0, 9.0, 9.1), _row(70, 20, "decode_b1", 10.2, 9.2, 9.2), _row(70, 20, "prefill_b1", 4.0, 5.0, 5.05)]
    cells = bench_request.aggregate(rows)
    decode = next(c for c in cells if c["shape"] == "decode_b1")
    assert decode["sessions"] == 2 and decode["ms"]["dense"] == pytest.approx(10.1)
    assert decode["hffn_over_dense"] == pytest.approx((0.9 + 9.2 / 10.2) / 2)
    judged = bench_request.admissibility(cells, complete=True, gate_passed=True)
    assert judged["admissible"] and judged["aa_values"] == 3
    shaky = bench_request.aggregate(rows + [_row(70, 20, "prefill_b4", 4.0, 5.0, 5.5)])
    assert not bench_request.admissibility(shaky, complete=True, gate_passed=True)["admissible"]  # 3 of 4 within 3 %
    assert not bench_request.admissibility(cells, complete=True, gate_passed=False)["admissible"]
    assert not bench_request.admissibility(cells, complete=False, gate_passed=True)["admissible"]


def test_block_order_goes_there_and_back():
    assert bench_request.block_order(0, 0) == ("hffn", "dense", "hffn_copy", "hffn_copy", "dense", "hffn")
    assert bench_request.block_order(1, 0) == bench_request.block_order(0, 1) == ("hffn_copy", "dense", "hffn", "hffn", "dense", "hffn_copy")


def _cpu_adapter():
    load = lambda model_dir, export_dir, ffn, device: pythia.load_pythia(model_dir, export_dir, ffn, "cpu",  # noqa: E731
                                                                         make_runtime=DenseStandIn)
    return bench_request.Adapter(name="CPU stand-in", load_pythia=load, device="cpu", synchronize=lambda: None,
                                 state=lambda: {"device": "cpu"}, versions=lambda: "test", describe=lambda model: {})


def test_campaign_order_and_files(tmp_path):
    seen = []

    def launcher(cell):
        seen.append(cell)
        row = {"size": cell.size, "density": cell.density, "shape": cell.shape, "gate_passed": True, "repeats": 3,
               "samples_ms": {arm: [1.0, 1.0] for arm in bench_request.ARMS}}
        return 0, "a log line\n" + json.dumps(row) + "\n", ""

    campaign = bench_request.Campaign(_cpu_adapter(), "smoke", tmp_path / "assets", tmp_path / "out", sessions=2, launcher=launcher)
    assert campaign.run() == 0
    assert [(c.session, c.shape, c.parity) for c in seen] == [(0, "prefill_b1", 0), (0, "decode_b1", 1), (1, "decode_b1", 0),
                                                              (1, "prefill_b1", 1)]
    for name in ("config.json", "provenance.json", "manifest.json", "raw.jsonl", "summary.json", "REPORT.md"):
        assert (tmp_path / "out" / name).exists(), name
    summary = json.loads((tmp_path / "out" / "summary.json").read_text())
    assert summary["verdict"]["admissible"] and len(summary["cells"]) == 2
    assert json.loads((tmp_path / "out" / "manifest.json").read_text())["status"] == "passed"


def test_campaign_stops_on_a_failed_gate(tmp_path):
    def launcher(cell):
        row = {"size": cell.size, "density": cell.density, "shape": cell.shape, "gate_passed": False, "repeats": None,
               "samples_ms": {arm: [] for arm in bench_request.ARMS}}
        return bench_request.GATE_FAILED, json.dumps(row), ""

    assert bench_request.Campaign(_cpu_adapter(), "smoke", tmp_path, tmp_path / "out", launcher=launcher).run() == 1
    summary = json.loads((tmp_path / "out" / "summary.json").read_text())
    assert summary["failure"]["returncode"] == bench_request.GATE_FAILED and summary["verdict"] is None


def test_one_cell_on_a_tiny_model(tmp_path):
    assert bench_request.prepare(tmp_path, {1: TINY}, [50])
    assert bench_request.prepare(tmp_path, {1: TINY}, [50]) == []  # nothing missing the second time
    cell = bench_request.Cell(size=1, density=50, shape="decode_b1", session=0, parity=1, blocks=1, window_ms=1.0, assets=str(tmp_path))
    row = bench_request.run_cell(_cpu_adapter(), cell)
    assert row["gate_passed"] and row["bitwise_copy"] and row["hffn_vs_dense_relative_gap"] <= bench_request.GUARD
    assert all(len(row["samples_ms"][arm]) == 2 and min(row["samples_ms"][arm]) > 0 for arm in bench_request.ARMS)  # both directions
    assert "assets" not in row
