"""Isolated-layer timing, HFFN against a dense iso-support control, with a copy of each arm for A/A admissibility: the
protocol of ``runtime/gpu/nvidia/ffn/inference/bench/bench_ffn.py`` (its constants: cells, grid, the two block orders,
the 2e-5 gate, the 3 % A/A criterion; ``runtime/common/ffn/hffn_ffn_layers/dense.py:14-39`` for the dense arm).

    python -m hffn_amd.bench_ffn --mode smoke|run [--cells pythia410m_d50:2048,pythia1p4b_d20_bf16:16] [--out FILE]

Arms: ``hffn`` and ``hffn_copy`` (two ``HFFNRuntime`` of the same layer), ``dense`` and ``dense_copy`` (PyTorch
``F.linear -> gelu -> F.linear`` in float32 on dense weights holding the support's values and zeros elsewhere). One
fresh process per session (``--worker``), all cells in it. A window is ``repeats`` calls of one arm on one resident
input between two synchronisations (host wall time), after an untimed window of the same arm; a block is eight
windows in one of the two orders, each arm twice with equal time centroid. Per cell: every arm's output within 2e-5
of the float64 dense result computed here, the copies bitwise equal, memory steady. A/A: every cell-session's
hffn/hffn_copy and dense/dense_copy ratio of medians within 3 %, else the session grid is not admissible and no ratio
is read. One JSON line per cell and a summary line.
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


def window(fn, repeats: int) -> float:
    """Milliseconds of `repeats` calls between two synchronisations."""
    import torch
    torch.cuda.synchronize()
    start = time.perf_counter_ns()
    for _ in range(repeats):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter_ns() - start) / 1e6


def worker(job: dict) -> int:
    import torch
    import torch.nn.functional as F

    from .ffn import hip_layer
    from .runtime import HFFNRuntime

    device = torch.device("cuda", 0)
    print(json.dumps({"event": "session", "session": job["session"]}), flush=True)
    with torch.inference_mode():
        for name, n in job["cells"]:
            layer, case, make_input = load_cell(name)
            x_np = make_input(case, n)
            x = torch.from_numpy(x_np).to(device)
            w_up, w_down = dense_weights(layer)
            expected = torch.from_numpy(float64_forward(layer, x_np, w_up, w_down)).to(device)

            def dense_arm():
                wu, wd = torch.from_numpy(w_up).to(device), torch.from_numpy(w_down).to(device)
                bu, bd = torch.from_numpy(layer.b_up.copy()).to(device), torch.from_numpy(layer.b_down.copy()).to(device)
                return lambda: F.linear(F.gelu(F.linear(x, wu, bu), approximate="none"), wd, bd)

            runtimes = [HFFNRuntime([hip_layer(layer, device)], device) for _ in range(2)]
            arms = {"dense": dense_arm(), "dense_copy": dense_arm(),
                    "hffn": lambda: runtimes[0].forward(0, x), "hffn_copy": lambda: runtimes[1].forward(0, x)}
            outputs = {arm: fn().clone() for arm, fn in arms.items()}
            scale = float(expected.abs().max().clamp(min=1.0))
            errors = {arm: float((y.double() - expected).abs().max()) / scale for arm, y in outputs.items()}
            gates = {"oracle": all(e <= TOLERANCE for e in errors.values()),
                     "copy_bitwise": bool(torch.equal(outputs["hffn"], outputs["hffn_copy"]))}
            for _ in range(3):
                for fn in arms.values():
                    fn()
            torch.cuda.synchronize()
            allocated = torch.cuda.memory_allocated()
            once = min(window(arms["dense"], 1) for _ in range(3))
            repeats = min(MAX_REPEATS, max(1, math.ceil(job["window_ms"] / once)))
            samples = {arm: [] for arm in arms}
            for order in BLOCK_ORDERS:
                for arm in order:
                    window(arms[arm], repeats)  # untimed lead-in of the same arm
                    samples[arm].append(window(arms[arm], repeats) / repeats * 1e3)  # µs per call
            gates["memory_steady"] = torch.cuda.memory_allocated() == allocated
            print(json.dumps({"event": "cell", "session": job["session"], "layer": name, "n": n, "repeats": repeats,
                              "samples_us": samples, "errors": errors, "gates": gates, "modes": list(runtimes[0].modes(n)),
                              "model_bytes": runtimes[0].layers[0].model_bytes(),
                              "dense_weight_bytes": 4 * 2 * layer.d_model * layer.d_ff}), flush=True)
            del arms, runtimes, outputs
            torch.cuda.empty_cache()
    print(json.dumps({"event": "session_end", "session": job["session"]}), flush=True)
    return 0


def median_ratio(samples: dict, a: str, b: str) -> float:
    return statistics.median(samples[a]) / statistics.median(samples[b])


def summarise(cells: list[dict]) -> dict:
    """A/A verdict over every cell-session, then (when admissible) the HFFN/dense ratios per cell."""
    aa = {pair: [median_ratio(c["samples_us"], pair, f"{pair}_copy") for c in cells] for pair in ("hffn", "dense")}
    verdict = {pair: {"within": sum(abs(v - 1) <= AA_TOLERANCE for v in values), "of": len(values),
                      "max_abs_dev": round(max((abs(v - 1) for v in values), default=1.0), 4)} for pair, values in aa.items()}
    gates = all(all(c["gates"].values()) for c in cells)
    admissible = bool(cells) and gates and all(v["within"] == v["of"] for v in verdict.values())
    rows = {}
    for c in cells:
        rows.setdefault((c["layer"], c["n"]), []).append(c)
    out = []
    for (layer, n), entries in rows.items():
        row = {"layer": layer, "n": n, "sessions": len(entries), "modes": entries[0]["modes"]}
        if admissible:
            ratios = [median_ratio(e["samples_us"], "hffn", "dense") for e in entries]
            row["hffn_over_dense"] = {"median": round(statistics.median(ratios), 4), "min": round(min(ratios), 4),
                                      "max": round(max(ratios), 4)}
            row["hffn_us"] = round(statistics.median(statistics.median(e["samples_us"]["hffn"]) for e in entries), 2)
            row["dense_us"] = round(statistics.median(statistics.median(e["samples_us"]["dense"]) for e in entries), 2)
        out.append(row)
    return {"event": "summary", "aa": verdict, "gates": gates, "admissible": admissible, "cells": out}


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
                                     | {"median_us": {a: round(statistics.median(v), 2) for a, v in record["samples_us"].items()}}),
                          flush=True)
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
