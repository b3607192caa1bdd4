"""Request-level timing of Pythia inference: the HFFN arm (FFNs on the HIP runtime), the dense arm (the same model with
dense iso-support FFNs) and a second HFFN instance (A/A), with the protocol of the reference's shared harness
(``runtime/common/pythia/hffn_pythia/bench_request.py:1-291``) and an MI355X adapter (the reference leaf's is
``runtime/gpu/nvidia/llm/inference/bench/bench_request.py``).

Protocol: one fresh process per cell (model size, density, request shape) holding three models loaded by
``hffn_amd.pythia.load_pythia`` that share one copy of the non-FFN weights; a window is a fixed number of consecutive
requests between two synchronisations, sized so that a dense window lasts at least ``window_ms``; every timed window
follows an untimed window of the same arm; arms run in both orders in every process. Gates before timing: the logits
of ``hffn_copy`` are bitwise those of ``hffn``, and ``hffn`` is within GUARD of max|logit| of ``dense``. A run is
admissible when at least AA_SHARE of the ratios ``hffn_copy / hffn`` (one per cell and session) lie within
1 +- AA_TOLERANCE; only then is ``hffn / dense`` read.

Models are random-init Pythia-shaped checkpoints with synthetic exports (``--prepare`` writes the missing ones) and the
prompts are synthetic tokens: the reference's checkpoints and WikiText-2 tokens are not available offline.

    python -m hffn_amd.bench_request --mode smoke|run --assets DIR --out DIR [--prepare] [--densities 10,50]
                                     [--sessions N] [--sizes 70,410]
    python -m hffn_amd.bench_request --worker '<cell json>'      (one cell in a fresh process, prints one JSON line)
"""
from __future__ import annotations

import argparse
import hashlib
import json
import statistics
import subprocess
import sys
import time
from dataclasses import dataclass, field
from datetime import datetime, timezone
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
ARMS = ("hffn", "dense", "hffn_copy")
SHAPES = {  # batch, prompt tokens, cached decode steps after the prompt call (bench_request.py:36-41)
    "prefill_b1": dict(batch=1, prompt=128, steps=0),
    "prefill_b4": dict(batch=4, prompt=128, steps=0),
    "decode_b1": dict(batch=1, prompt=32, steps=16),
    "decode_b4": dict(batch=4, prompt=32, steps=16),
}
GRID = {  # sizes, densities, shapes, sessions, blocks, minimum window of the dense arm in ms (bench_request.py:42-45)
    "run": dict(sizes=(70, 160, 410), densities=(10, 20, 50, 80), shapes=tuple(SHAPES), sessions=3, blocks=2, window_ms=300.0),
    "smoke": dict(sizes=(70,), densities=(20,), shapes=("prefill_b1", "decode_b1"), sessions=1, blocks=1, window_ms=60.0),
}
GUARD = 1e-3              # hffn against dense, as a fraction of max|logit|
AA_TOLERANCE, AA_SHARE = 0.03, 0.95
MAX_REPEATS = 200
SIZES = {  # Pythia family shapes (GPT-NeoX configs of EleutherAI/pythia-70m, -160m, -410m)
    70: dict(hidden_size=512, num_hidden_layers=6, num_attention_heads=8, intermediate_size=2048),
    160: dict(hidden_size=768, num_hidden_layers=12, num_attention_heads=12, intermediate_size=3072),
    410: dict(hidden_size=1024, num_hidden_layers=24, num_attention_heads=16, intermediate_size=4096),
}
SEED = 104


def folders(assets: Path, size, density: int) -> tuple[Path, Path]:
    return Path(assets) / f"pythia{size}m", Path(assets) / f"pythia{size}m_sparse{density}" / "export"


def prepare(assets: Path, sizes: dict, densities) -> list[str]:
    """Write the missing random-init checkpoints (one per size) and exports (one per size and density)."""
    from . import pythia
    written = []
    for size, overrides in sizes.items():
        model_dir, _ = folders(assets, size, 0)
        if not (model_dir / "model.safetensors").exists():
            pythia.write_random_checkpoint(model_dir, SEED, **overrides)
            written.append(str(model_dir))
        config = pythia.pythia_config(**overrides)
        for density in densities:
            _, export_dir = folders(assets, size, density)
            if not pythia.layer_path(export_dir, 0).exists():
                pythia.write_random_exports(export_dir, config, density / 100, SEED)
                written.append(str(export_dir))
    return written


@dataclass
class Adapter:
    """What a hardware leaf gives the harness (``bench_request.py:50-70`` of the reference): its loader, where the
    prompt tensors live, how to wait for queued work, what to record of the device, versions, what it reports of its
    HFFN runtime after a cell, and the files hashed in the provenance."""
    name: str
    load_pythia: object
    device: str
    synchronize: object
    state: object
    versions: object
    describe: object
    runtime_files: list = field(default_factory=list)
    note: str = ""


def _hip_state() -> dict:
    import torch
    if not torch.cuda.is_available():
        return {"device": "none"}
    free, total = torch.cuda.mem_get_info()
    return {"device": torch.cuda.get_device_name(0), "memory_used": total - free, "time": time.time()}


def _hip_versions() -> str:
    import torch
    import transformers
    return f"python {sys.version.split()[0]} torch {torch.__version__} hip {torch.version.hip} transformers {transformers.__version__}"


def _hip_describe(model) -> dict:
    import torch
    runtime = model.hffn_runtime
    return {"kernels": {f"{up}/{down}": count for (up, down), count in sorted(runtime.calls.items())},
            "workspace_bytes": runtime.workspace_bytes(), "max_memory_allocated": torch.cuda.max_memory_allocated()}


def hip_adapter() -> Adapter:
    import torch

    from . import pythia
    files = sorted((ROOT / "hffn_amd" / "csrc").glob("*")) + sorted((ROOT / "hffn_amd").glob("*.py")) + [ROOT / "include" / "hffn_amd.h"]
    return Adapter(name="MI355X HIP leaf", load_pythia=pythia.load_pythia, device="cuda", synchronize=torch.cuda.synchronize,
                   state=_hip_state, versions=_hip_versions, describe=_hip_describe, runtime_files=files,
                   note="one MI355X per box: ratios hold within one execution only")


def sha256(path: Path) -> str:
    digest = hashlib.sha256()
    with open(path, "rb") as stream:
        for chunk in iter(lambda: stream.read(1 << 20), b""):
            digest.update(chunk)
    return digest.hexdigest()


# -- worker ---------------------------------------------------------------------------------------------------------

def worker(adapter: Adapter, cell: dict) -> dict:
    """Gates and timed windows of one cell (``bench_request.py:97-170``); returns the row (also printed by main)."""
    import torch

    from . import pythia
    model_dir, export_dir = folders(Path(cell["assets"]), cell["size"], cell["density"])
    load = adapter.load_pythia
    models = {"dense": load(model_dir, export_dir, "dense", adapter.device), "hffn": load(model_dir, export_dir, "hffn", adapter.device),
              "hffn_copy": load(model_dir, export_dir, "hffn", adapter.device)}
    for arm in ("hffn", "hffn_copy"):  # one copy of the non-FFN weights: the arms differ by the FFN only
        pythia.share_non_ffn(models[arm], models["dense"])
    shape = SHAPES[cell["shape"]]
    batch, length, steps = shape["batch"], shape["prompt"], shape["steps"]
    prompt = pythia.synthetic_prompts(batch, length, models["dense"].config.vocab_size).to(adapter.device)

    def request(arm, tokens, keep=False):
        """One request: the prompt call, then the cached decode steps fed with `tokens`. No synchronisation. With
        `keep`, the last-position logits of every call."""
        model = models[arm]
        out = model(input_ids=prompt, use_cache=True)
        logits = [out.logits[:, -1].clone()] if keep else None
        for token in tokens:
            out = model(input_ids=token, past_key_values=out.past_key_values, use_cache=True)
            if keep:
                logits.append(out.logits[:, -1].clone())
        return logits

    def window(arm, tokens, repeats):
        adapter.synchronize()
        start = time.perf_counter_ns()
        for _ in range(repeats):
            request(arm, tokens)
        adapter.synchronize()
        return (time.perf_counter_ns() - start) / repeats / 1e6

    with torch.inference_mode():
        out = models["dense"](input_ids=prompt, use_cache=True)  # greedy tokens of the dense arm, fed to every arm
        tokens = []
        for _ in range(steps):
            tokens.append(out.logits[:, -1:].argmax(-1))
            out = models["dense"](input_ids=tokens[-1], past_key_values=out.past_key_values, use_cache=True)
        del out
        reference = {arm: request(arm, tokens, keep=True) for arm in ARMS}
        bitwise = all(bool(torch.equal(a, b)) for a, b in zip(reference["hffn_copy"], reference["hffn"]))
        pairs = list(zip(reference["hffn"], reference["dense"]))
        gap = max(float((a - b).abs().max()) for a, b in pairs) / max(float(b.abs().max()) for _, b in pairs)
        argmax_differ = sum(int((a.argmax(-1) != b.argmax(-1)).sum()) for a, b in pairs)
        del reference, pairs
        passed = bitwise and gap <= GUARD
        samples, repeats = {arm: [] for arm in ARMS}, None
        if passed:
            for arm in ARMS:  # warm-up: buffers reserved, kernels loaded
                window(arm, tokens, 2)
            once = min(window("dense", tokens, 1) for _ in range(3))
            repeats = max(1, min(MAX_REPEATS, int(cell["window_ms"] / once) + 1))
            orders = (ARMS + ARMS[::-1], ARMS[::-1] + ARMS)
            for block in range(cell["blocks"]):
                for arm in orders[(cell["parity"] + block) % 2]:
                    window(arm, tokens, repeats)  # untimed window of the same arm before each timed one
                    samples[arm].append(window(arm, tokens, repeats))
    return {**{k: v for k, v in cell.items() if k != "assets"}, "samples_ms": samples, "repeats": repeats, "bitwise_copy": bitwise,
            "hffn_vs_dense_relative_gap": gap, "argmax_differing_positions": argmax_differ, "gate_passed": passed,
            "runtime": adapter.describe(models["hffn"])}


# -- orchestrator ---------------------------------------------------------------------------------------------------

def summarize(rows: list[dict]) -> list[dict]:
    """Per cell: median ms per arm over sessions, the hffn/dense ratio (median, min, max) and the A/A ratios."""
    cells: dict = {}
    for row in rows:
        cells.setdefault((row["size"], row["density"], row["shape"]), []).append(
            {arm: statistics.median(row["samples_ms"][arm]) for arm in ARMS})
    out = []
    for (size, density, shape), values in sorted(cells.items(), key=lambda item: tuple(str(k) for k in item[0])):
        ratio = [v["hffn"] / v["dense"] for v in values]
        out.append({"size": size, "density": density, "shape": shape, "sessions": len(values),
                    "ms": {arm: statistics.median(v[arm] for v in values) for arm in ARMS},
                    "hffn_over_dense": statistics.median(ratio), "min": min(ratio), "max": max(ratio),
                    "aa": [v["hffn_copy"] / v["hffn"] for v in values]})
    return out


def verdict(cells: list[dict], complete: bool, gate_passed: bool) -> dict:
    """Admissibility, fixed before any measurement (``bench_request.py:187-196``)."""
    if not complete:
        return {"admissible": False, "reason": "incomplete coverage"}
    aa = [a for c in cells for a in c["aa"]]
    inside = sum(abs(a - 1) <= AA_TOLERANCE for a in aa)
    return {"admissible": gate_passed and inside >= AA_SHARE * len(aa), "gate_passed": gate_passed, "aa_values": len(aa),
            "aa_within_tolerance": inside, "aa_share": inside / len(aa), "aa_median": statistics.median(aa),
            "aa_min": min(aa), "aa_max": max(aa)}


def cells_of(grid: dict) -> list[dict]:
    return [dict(size=s, density=d, shape=shape) for s in grid["sizes"] for d in grid["densities"] for shape in grid["shapes"]]


def report_lines(adapter_name: str, mode: str, done: int, planned: int, cells: list[dict], judged, failed) -> list[str]:
    status = "passed" if done == planned else "failed"
    lines = [f"# Request-level harness, {adapter_name}, {mode}", "", f"Status: {status}; {done}/{planned} processes.", "",
             "Milliseconds per request. `hffn/dense` is read only if the verdict below says admissible.", "",
             "| model | density | shape | dense | hffn | hffn/dense [min-max] | A/A per session |", "|---|---:|---|---:|---:|---|---|"]
    for c in cells:
        lines.append(f"| {c['size']}M | {c['density']} % | {c['shape']} | {c['ms']['dense']:.3f} | {c['ms']['hffn']:.3f} | "
                     f"{c['hffn_over_dense']:.3f} [{c['min']:.3f}-{c['max']:.3f}] | " + " ".join(f"{a:.3f}" for a in c["aa"]) + " |")
    lines += ["", "```json", json.dumps(judged, indent=1), "```"]
    if failed:
        lines += ["", "Failure:", "```", json.dumps(failed, indent=1)[:4000], "```"]
    return lines


def orchestrate(adapter: Adapter, mode: str, assets: Path, out: Path, densities=None, sessions=None, sizes=None,
                run_cell=None) -> int:
    """Every cell of the grid in a fresh process per session (cells in alternating order), then the summary, the
    verdict and REPORT.md in `out`. `run_cell(job) -> (returncode, stdout, stderr)` replaces the subprocess (tests)."""
    grid = {**GRID[mode], **({"densities": tuple(densities)} if densities else {}), **({"sessions": sessions} if sessions else {}),
            **({"sizes": tuple(sizes)} if sizes else {})}
    cells = cells_of(grid)
    planned = len(cells) * grid["sessions"]
    out.mkdir(parents=True, exist_ok=True)
    (out / "config.json").write_text(json.dumps({"mode": mode, **grid, "arms": ARMS, "shape_definitions": SHAPES, "guard": GUARD,
                                                 "aa_tolerance": AA_TOLERANCE, "aa_share": AA_SHARE}, indent=1) + "\n")
    (out / "provenance.json").write_text(json.dumps({
        "leaf": adapter.name, "runtime_files": {str(Path(p).relative_to(ROOT)): sha256(Path(p)) for p in adapter.runtime_files},
        "versions": adapter.versions(), "state_at_start": adapter.state(), "machine": adapter.note}, indent=1) + "\n")
    manifest = {"status": "running", "planned": planned, "done": 0, "started": datetime.now(timezone.utc).isoformat()}
    write = lambda: (out / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")  # noqa: E731
    write()
    if run_cell is None:
        def run_cell(job):
            result = subprocess.run([sys.executable, "-B", "-m", "hffn_amd.bench_request", "--worker", json.dumps(job)],
                                    text=True, capture_output=True, cwd=ROOT)
            return result.returncode, result.stdout, result.stderr
    rows, failed = [], None
    with (out / "raw.jsonl").open("w") as raw:
        for session in range(grid["sessions"]):
            order = list(enumerate(cells)) if session % 2 == 0 else list(enumerate(cells))[::-1]
            for index, cell in order:
                job = {**cell, "session": session, "parity": (session + index) % 2, "blocks": grid["blocks"],
                       "window_ms": grid["window_ms"], "assets": str(assets)}
                state = adapter.state()
                code, stdout, stderr = run_cell(job)
                lines = [line for line in stdout.strip().splitlines() if line.startswith("{")]
                if code not in (0, 4) or not lines:
                    failed = {"cell": cell, "session": session, "returncode": code, "stderr": stderr[-4000:]}
                    break
                row = {**json.loads(lines[-1]), "state_before": state}
                raw.write(json.dumps(row) + "\n")
                raw.flush()
                rows.append(row)
                if code == 4:
                    failed = {"cell": cell, "session": session, "returncode": 4, "row": {k: v for k, v in row.items() if k != "samples_ms"}}
                    break
                manifest["done"] += 1
                write()
                med = {arm: statistics.median(row["samples_ms"][arm]) for arm in ARMS}
                print(f"[{manifest['done']}/{planned}] s{session} pythia{cell['size']}m d{cell['density']} {cell['shape']} "
                      f"x{row['repeats']}: " + ", ".join(f"{arm} {med[arm]:.3f}" for arm in ARMS) + " ms", flush=True)
            if failed:
                break
    complete = manifest["done"] == planned
    gate_passed = failed is None or failed["returncode"] != 4
    summary_cells = summarize(rows) if complete else []
    judged = verdict(summary_cells, complete, gate_passed) if summary_cells else None
    (out / "summary.json").write_text(json.dumps({"cells": summary_cells, "verdict": judged, "failure": failed,
                                                  "state_at_end": adapter.state()}, indent=1) + "\n")
    report = report_lines(adapter.name, mode, manifest["done"], planned, summary_cells, judged, failed)
    (out / "REPORT.md").write_text("\n".join(report) + "\n")
    manifest.update(status="passed" if complete else "failed", finished=datetime.now(timezone.utc).isoformat())
    write()
    print("\n".join(report), flush=True)
    return 0 if complete else 1


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--worker")
    parser.add_argument("--mode", choices=sorted(GRID))
    parser.add_argument("--assets", type=Path, help="holds pythia<size>m/ checkpoints and pythia<size>m_sparse<d>/export/")
    parser.add_argument("--prepare", action="store_true", help="write the missing random-init checkpoints and exports first")
    parser.add_argument("--out", type=Path)
    parser.add_argument("--densities", type=lambda text: tuple(int(v) for v in text.split(",")), default=None)
    parser.add_argument("--sessions", type=int, default=None)
    parser.add_argument("--sizes", type=lambda text: tuple(int(v) for v in text.split(",")), default=None)
    args = parser.parse_args(argv)
    adapter = hip_adapter()
    if args.worker:
        row = worker(adapter, json.loads(args.worker))
        print(json.dumps(row), flush=True)
        return 0 if row["gate_passed"] else 4
    if not args.mode or not args.assets or not args.out:
        parser.error("--mode, --assets and --out are required")
    grid = GRID[args.mode]
    sizes = args.sizes or grid["sizes"]
    densities = args.densities or grid["densities"]
    if args.prepare:
        for path in prepare(args.assets, {s: SIZES[s] for s in sizes}, densities):
            print(f"wrote {path}", flush=True)
    missing = [str(f) for s in sizes for d in densities for f in (folders(args.assets, s, d)[0] / "model.safetensors",
                                                                  folders(args.assets, s, d)[1] / "layer0") if not f.exists()]
    if missing:
        raise SystemExit(f"missing assets (use --prepare): {missing}")
    return orchestrate(adapter, args.mode, args.assets, args.out, args.densities, args.sessions, args.sizes)


if __name__ == "__main__":
    sys.exit(main())
