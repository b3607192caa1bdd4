"""The request-level harness end to end on the GPU: a smoke grid on a tiny random-init Pythia, every cell in a fresh
process with the HIP adapter, gates passed and a verdict written."""
from __future__ import annotations

import json

import pytest

from hffn_amd import bench_request
from tests.test_pythia import TINY

pytestmark = pytest.mark.gpu


def test_smoke_grid_on_a_tiny_model(tmp_path, device):
    bench_request.prepare(tmp_path / "assets", {1: TINY}, [50])
    out = tmp_path / "out"
    code = bench_request.Campaign(bench_request.hip_adapter(), "smoke", tmp_path / "assets", out, densities=[50], sizes=[1]).run()
    summary = json.loads((out / "summary.json").read_text())
    assert code == 0, summary["failure"]
    assert summary["verdict"]["gate_passed"] and len(summary["cells"]) == 2
    rows = [json.loads(line) for line in (out / "raw.jsonl").read_text().splitlines()]
    assert all(row["bitwise_copy"] and row["runtime"]["kernels"] for row in rows)
    assert (out / "REPORT.md").read_text().startswith("# Request-level harness, MI355X HIP leaf, smoke")
