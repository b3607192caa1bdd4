"""Isolated-layer timing, HFFN against a dense iso-support control, with a copy of each arm for A/A admissibility: the
protocol of ``runtime/gpu/nvidia/ffn/inference/bench/bench_ffn.py`` (its constants: cells, grid, the two block orders,
the 2e-5 gate, the 3 % A/A criterion; ``runtime/common/ffn/hffn_ffn_layers/dense.py:14-39`` for the dense arm).

    python -m hffn_amd.bench_ffn --mode smoke|run [--cells pythia410m_d50:2048,pythia1p4b_d20_bf16:16] [--out FILE]

Arms: ``hffn`` and ``hffn_copy`` (two ``HFFNRuntime`` of the same layer), ``dense`` and ``dense_copy`` (PyTorch
``F.linear -> gelu -> F.linear`` in float32 on dense weights holding the support's values and zeros elsewhere). One
fresh process per session (``--worker``), all cells in it. A window is ``repeats`` calls of one arm on one resident
input between two synchronisations (host wall time), after an untimed window of the same arm; a block is eight
windows in one of the two orders, each arm twice with equal time centroid. ``repeats`` makes the slowest arm's window
last the grid's window time. The worker reports every timed window as one observation (block, slot, arm, µs); the
summary groups them. Per cell: every arm's output within 2e-5 of the float64 dense result computed here, the copies
bitwise equal, memory steady. A/A: every cell-session's hffn/hffn_copy and dense/dense_copy ratio of medians within
3 %, else the session grid is not admissible and no ratio is read. One JSON line per cell and a summary line.
"""
from __future__ import annotations

import argparse
import json
import math
import statistics
import subprocess
import sys
import time

import numpy as np

CELLS = {
    "run": (("homog_512_2048", 1), ("homog_512_2048", 4), ("homog_512_2048", 64), ("homog_512_2048", 512),
            ("irreg_512_2048", 4), ("irreg_512_2048", 512)),
    "smoke": (("homog_512_2048", 1), ("homog_512_2048", 64)),
}
GRID = {"run": dict(sessions=3, window_ms=50.0), "smoke": dict(sessions=1, window_ms=20.0)}
BLOCK_ORDERS = (("dense", "hffn", "hffn_copy", "dense_copy", "dense_copy", "hffn_copy", "hffn", "dense"),
                ("dense_copy", "hffn_copy", "hffn", "dense", "dense", "hffn", "hffn_copy", "dense_copy"))
TOLERANCE = 2e-5
AA_TOLERANCE = 0.03
MAX_REPEATS = 100_000


def dense_weights(layer) -> tuple[np.ndarray, np.ndarray]:
    """W_up [d_ff, d_model] and W_down [d_model, d_ff] (float32) with the support's values and zeros elsewhere."""
    rows_up = np.repeat(np.arange(layer.d_ff), np.diff(layer.up_offsets))
    rows_down = np.repeat(np.arange(layer.d_ff), np.diff(layer.down_offsets))
    w_up = np.zeros((layer.d_ff, layer.d_model), np.float32)
    w_down = np.zeros((layer.d_model, layer.d_ff), np.float32)
    w_up[rows_up, layer.up_idx.astype(np.int64) & 0xFFFF] = layer.up_val
    w_down[layer.down_idx.astype(np.int64) & 0xFFFF, rows_down] = layer.down_val
    return w_up, w_down


def float64_forward(layer, x: np.ndarray, w_up: np.ndarray, w_down: np.ndarray) -> np.ndarray:
    """The dense layer in float64 (exact-erf GELU): the gate every arm's output is held to."""
    from scipy.special import erf
    z = x.astype(np.float64) @ w_up.T.astype(np.float64) + layer.b_up
    return (0.5 * z * (1.0 + erf(z / math.sqrt(2.0)))) @ w_down.T.astype(np.float64) + layer.b_down


def load_cell(name: str):
    from . import synth
    if name in synth.CASES:
        case = synth.CASES[name]
        return synth.make_layer(case), case, synth.make_input
    workload = synth.WORKLOADS[name]
    return synth.make_workload_layer(workload), workload, synth.make_input


ARMS = ("hffn", "hffn_copy", "dense", "dense_copy")


def schedule() -> list[tuple[int, int, str]]:
    """(block, slot, arm) of every timed window of a cell: the blocks of ``BLOCK_ORDERS`` one after the other."""
    return [(block, slot, arm) for block, order in enumerate(BLOCK_ORDERS) for slot, arm in enumerate(order)]


class LayerCell:
    """One (layer, N) cell in a worker: the input on the device, its float64 expectation, and the four arms as
    callables (two HFFNRuntime of the same layer; two dense iso-support PyTorch layers)."""

    def __init__(self, name: str, n: int, device) -> None:
        import torch
        import torch.nn.functional as F

        from .ffn import hip_layer
        from .runtime import HFFNRuntime

        self.name, self.n = name, n
        layer, case, make_input = load_cell(name)
        x_np = make_input(case, n)
        w_up, w_down = dense_weights(layer)
        self.expected = torch.from_numpy(float64_forward(layer, x_np, w_up, w_down)).to(device)
        self.x = torch.from_numpy(x_np).to(device)
        self.runtimes = [HFFNRuntime([hip_layer(layer, device)], device) for _ in range(2)]
        dense = [tuple(torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in (w_up, layer.b_up, w_down, layer.b_down))
                 for _ in range(2)]
        x = self.x
        self.arms = {
            "hffn": lambda: self.runtimes[0].forward(0, x),
            "hffn_copy": lambda: self.runtimes[1].forward(0, x),
            "dense": lambda p=dense[0]: F.linear(F.gelu(F.linear(x, p[0], p[1]), approximate="none"), p[2], p[3]),
            "dense_copy": lambda p=dense[1]: F.linear(F.gelu(F.linear(x, p[0], p[1]), approximate="none"), p[2], p[3]),
        }
        self.record = {"layer": name, "n": n, "modes": list(self.runtimes[0].modes(n)),
                       "model_bytes": self.runtimes[0].layers[0].model_bytes(),
                       "workspace_bytes": self.runtimes[0].workspace_bytes(),
                       "dense_weight_bytes": 4 * 2 * layer.d_model * layer.d_ff}

    def gates(self) -> dict:
        """Before any timing: every arm within TOLERANCE of the float64 layer (relative to max(1, max |y64|)), and the
        two HFFN runtimes bitwise equal."""
        import torch
        out = {arm: fn().clone() for arm, fn in self.arms.items()}
        scale = float(self.expected.abs().max().clamp(min=1.0))
        errors = {arm: float((y.double() - self.expected).abs().max()) / scale for arm, y in out.items()}
        self.record["errors"] = errors
        return {"oracle": max(errors.values()) <= TOLERANCE, "copy_bitwise": bool(torch.equal(out["hffn"], out["hffn_copy"]))}

    def window_us(self, arm: str, repeats: int) -> float:
        """µs per call over ``repeats`` calls of ``arm`` between two synchronisations (host wall clock)."""
        import torch
        fn = self.arms[arm]
        torch.cuda.synchronize()
        began = time.perf_counter_ns()
        for _ in range(repeats):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter_ns() - began) / repeats / 1e3

    def repeats_for(self, window_ms: float) -> int:
        """Calls per window: enough that the slowest arm's window lasts ``window_ms`` (its single-call time is the best
        of three after a warm-up call of every arm), so that no arm's window is shorter."""
        for arm in ARMS:
            self.window_us(arm, 1)
        slowest = max(min(self.window_us(arm, 1) for _ in range(3)) for arm in ARMS)
        return max(1, min(MAX_REPEATS, math.ceil(window_ms * 1e3 / slowest)))

    def observe(self, repeats: int) -> list[dict]:
        """The schedule's windows, each after an untimed window of the same arm: one observation per timed window."""
        rows = []
        for block, slot, arm in schedule():
            self.window_us(arm, repeats)
            rows.append({"block": block, "slot": slot, "arm": arm, "us": self.window_us(arm, repeats)})
        return rows


def worker(job: dict) -> int:
    """One session: every cell of the job in this process, one JSON line per cell (gates, then the observations)."""
    import torch
    device = torch.device("cuda", 0)
    print(json.dumps({"event": "session", "session": job["session"]}), flush=True)
    with torch.inference_mode():
        for name, n in job["cells"]:
            cell = LayerCell(name, n, device)
            gates = cell.gates()
            repeats = cell.repeats_for(job["window_ms"])
            torch.cuda.synchronize()
            held = torch.cuda.memory_allocated()
            observations = cell.observe(repeats)
            gates["memory_steady"] = torch.cuda.memory_allocated() == held
            print(json.dumps({"event": "cell", "session": job["session"], **cell.record, "repeats": repeats, "gates": gates,
                              "observations": observations}), flush=True)
            del cell
            torch.cuda.empty_cache()
    print(json.dumps({"event": "session_end", "session": job["session"]}), flush=True)
    return 0


def arm_medians(cell: dict) -> dict:
    """Median µs per call of each arm over a cell-session's observations."""
    by_arm: dict = {}
    for row in cell["observations"]:
        by_arm.setdefault(row["arm"], []).append(row["us"])
    return {arm: statistics.median(values) for arm, values in by_arm.items()}


def summarise(cells: list[dict]) -> dict:
    """Per cell-session, the arm medians; A/A (each arm over its copy) must hold within AA_TOLERANCE in every
    cell-session, and every gate must pass, before any HFFN/dense ratio is reported (median, min and max over the
    sessions of each cell)."""
    table = [{"key": (c["layer"], c["n"]), "modes": c["modes"], "gates": c["gates"], **arm_medians(c)} for c in cells]
    deviations = {pair: [abs(t[pair] / t[f"{pair}_copy"] - 1.0) for t in table] for pair in ("hffn", "dense")}
    aa = {pair: {"within": sum(d <= AA_TOLERANCE for d in devs), "of": len(devs), "max_abs_dev": round(max(devs, default=1.0), 4)}
          for pair, devs in deviations.items()}
    gates = all(all(t["gates"].values()) for t in table)
    admissible = bool(table) and gates and all(v["within"] == v["of"] for v in aa.values())
    keys = list(dict.fromkeys(t["key"] for t in table))
    rows = []
    for key in keys:
        sessions = [t for t in table if t["key"] == key]
        row = {"layer": key[0], "n": key[1], "sessions": len(sessions), "modes": sessions[0]["modes"]}
        if admissible:
            ratios = sorted(t["hffn"] / t["dense"] for t in sessions)
            row["hffn_over_dense"] = {"median": round(statistics.median(ratios), 4), "min": round(ratios[0], 4),
                                      "max": round(ratios[-1], 4)}
            row["hffn_us"] = round(statistics.median(t["hffn"] for t in sessions), 2)
            row["dense_us"] = round(statistics.median(t["dense"] for t in sessions), 2)
        rows.append(row)
    return {"event": "summary", "aa": aa, "gates": gates, "admissible": admissible, "cells": rows}


def parse_cells(text: str) -> list[tuple[str, int]]:
    cells = []
    for item in text.split(","):
        name, _, n = item.partition(":")
        cells.append((name, int(n)))
    return cells


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--mode", choices=sorted(GRID), default="smoke")
    parser.add_argument("--cells", help="cells instead of the mode's, e.g. pythia410m_d50:2048,pythia1p4b_d20_bf16:16")
    parser.add_argument("--sessions", type=int, help="sessions instead of the mode's")
    parser.add_argument("--out", help="also write every line here")
    parser.add_argument("--worker", help=argparse.SUPPRESS)
    args = parser.parse_args(argv)
    if args.worker:
        return worker(json.loads(args.worker))
    grid = dict(GRID[args.mode])
    cells = parse_cells(args.cells) if args.cells else list(CELLS[args.mode])
    sessions = args.sessions or grid["sessions"]
    lines = []
    for session in range(sessions):
        job = {"session": session, "cells": cells, "window_ms": grid["window_ms"]}
        result = subprocess.run([sys.executable, "-m", "hffn_amd.bench_ffn", "--worker", json.dumps(job)],
                                capture_output=True, text=True)
        for line in result.stdout.splitlines():
            if line.startswith("{"):
                record = json.loads(line)
                lines.append(record)
                if record["event"] == "cell":
                    print(json.dumps({k: record[k] for k in ("session", "layer", "n", "repeats", "gates", "modes")}
                                     | {"median_us": {a: round(v, 2) for a, v in arm_medians(record).items()}}), flush=True)
        if result.returncode != 0:
            print(result.stderr[-2000:], file=sys.stderr)
            return result.returncode
    summary = summarise([r for r in lines if r["event"] == "cell"])
    print(json.dumps(summary), flush=True)
    if args.out:
        with open(args.out, "w") as f:
            for record in lines + [summary]:
                f.write(json.dumps(record) + "\n")
    return 0 if summary["gates"] else 1


if __name__ == "__main__":
    raise SystemExit(main())
