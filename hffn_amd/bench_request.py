"""Request-level timing of Pythia inference with the HFFN arm on the HIP runtime.

The protocol is the reference's shared harness (``runtime/common/pythia/hffn_pythia/bench_request.py:1-20``, leaf
adapter ``runtime/gpu/nvidia/llm/inference/bench/bench_request.py``); the code is this package's own.

* A cell is (model size, density, request shape). Every cell runs in a fresh process per session, holding three arms
  built by ``load_pythia``: ``hffn``, ``dense`` (the same FFNs densified on their support) and ``hffn_copy`` (a second
  HFFN instance, the A/A control). The three read one copy of the non-FFN weights.
* A request is the prompt call and then the cached decode steps of the shape, fed with the dense arm's greedy tokens.
* Gates before any timing: ``hffn_copy`` gives bitwise the logits of ``hffn``; ``hffn`` is within ``GUARD`` of the
  largest dense logit.
* A window is ``repeats`` back-to-back requests between two synchronisations; ``repeats`` is fixed per cell so that a
  dense window lasts at least ``window_ms``. Each timed window follows an untimed one of the same arm, and each block
  visits the arms forwards then backwards (the starting direction alternates with the cell's parity and the block).
* The run is admissible when no gate failed and at least ``AA_SHARE`` of the ratios ``hffn_copy / hffn`` (one per
  cell and session) lie within ``1 +- AA_TOLERANCE``; only then is ``hffn / dense`` read.

The checkpoints are random-init Pythia shapes with synthetic exports (``--prepare`` writes what is missing) and the
prompts are synthetic tokens: the reference's assets are not available offline.

    python -m hffn_amd.bench_request --mode smoke|run --assets DIR --out DIR [--prepare] [--sizes 410] [--densities 50]
                                     [--sessions N]
    python -m hffn_amd.bench_request --worker '<cell json>'      (one cell; prints one JSON line, exit 4 on a failed gate)
"""
from __future__ import annotations

import argparse
import hashlib
import json
import statistics
import subprocess
import sys
import time
from dataclasses import asdict, dataclass, field
from datetime import datetime, timezone
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]

# -- protocol constants (bench_request.py:35-47 of the reference) ------------------------------------------------------
ARMS = ("hffn", "dense", "hffn_copy")
SHAPES = {  # batch, prompt tokens, cached decode steps after the prompt call
    "prefill_b1": dict(batch=1, prompt=128, steps=0),
    "prefill_b4": dict(batch=4, prompt=128, steps=0),
    "decode_b1": dict(batch=1, prompt=32, steps=16),
    "decode_b4": dict(batch=4, prompt=32, steps=16),
}
GRID = {  # sizes, densities, shapes, sessions, blocks per process, minimum dense window (ms)
    "run": dict(sizes=(70, 160, 410), densities=(10, 20, 50, 80), shapes=tuple(SHAPES), sessions=3, blocks=2, window_ms=300.0),
    "smoke": dict(sizes=(70,), densities=(20,), shapes=("prefill_b1", "decode_b1"), sessions=1, blocks=1, window_ms=60.0),
}
GUARD = 1e-3              # largest |hffn - dense| logit gap, as a fraction of the largest dense logit
AA_TOLERANCE, AA_SHARE = 0.03, 0.95
MAX_REPEATS = 200
GATE_FAILED = 4           # exit status of a worker whose gates failed

# Pythia family shapes (the GPT-NeoX configs of EleutherAI/pythia-70m, -160m and -410m).
SIZES = {
    70: dict(hidden_size=512, num_hidden_layers=6, num_attention_heads=8, intermediate_size=2048),
    160: dict(hidden_size=768, num_hidden_layers=12, num_attention_heads=12, intermediate_size=3072),
    410: dict(hidden_size=1024, num_hidden_layers=24, num_attention_heads=16, intermediate_size=4096),
}
SEED = 104


# -- assets -------------------------------------------------------------------------------------------------------------

def asset_dirs(assets: Path, size, density: int) -> tuple[Path, Path]:
    """(checkpoint folder, export folder) of one model size and density under ``assets``."""
    return Path(assets) / f"pythia{size}m", Path(assets) / f"pythia{size}m_sparse{density}" / "export"


def prepare(assets: Path, sizes: dict, densities) -> list[str]:
    """Write what is missing: one random-init checkpoint per size, one synthetic export per (size, density). Returns the
    folders written."""
    from . import pythia
    written = []
    for size, shape in sizes.items():
        checkpoint, _ = asset_dirs(assets, size, 0)
        if not (checkpoint / "model.safetensors").exists():
            pythia.write_random_checkpoint(checkpoint, SEED, **shape)
            written.append(str(checkpoint))
        for density in densities:
            _, export = asset_dirs(assets, size, density)
            if not pythia.layer_path(export, 0).exists():
                pythia.write_random_exports(export, pythia.pythia_config(**shape), density / 100, SEED)
                written.append(str(export))
    return written


# -- what a leaf provides -----------------------------------------------------------------------------------------------

@dataclass
class Adapter:
    """The hardware side of the harness (``bench_request.py:50-70`` of the reference): ``load_pythia(model_dir,
    export_dir, ffn, device)``, the device of the prompts, ``synchronize()``, ``state()`` (recorded before every
    process), ``versions()`` (one line), ``describe(model)`` (what the leaf reports of its HFFN runtime after a cell)
    and the files hashed into the provenance."""
    name: str
    load_pythia: object
    device: str
    synchronize: object
    state: object
    versions: object
    describe: object
    runtime_files: list = field(default_factory=list)
    note: str = ""


def _gpu_state() -> dict:
    import torch
    if not torch.cuda.is_available():
        return {"device": "none"}
    free, total = torch.cuda.mem_get_info()
    return {"device": torch.cuda.get_device_name(0), "memory_used": total - free, "time": time.time()}


def _versions() -> str:
    import torch
    import transformers
    return f"python {sys.version.split()[0]} torch {torch.__version__} hip {torch.version.hip} transformers {transformers.__version__}"


def _runtime_report(model) -> dict:
    import torch
    runtime = model.hffn_runtime
    return {"kernels": {f"{up}/{down}": count for (up, down), count in sorted(runtime.calls.items())},
            "workspace_bytes": runtime.workspace_bytes(), "max_memory_allocated": torch.cuda.max_memory_allocated()}


def hip_adapter() -> Adapter:
    import torch

    from . import pythia
    sources = [*sorted((ROOT / "hffn_amd" / "csrc").glob("*")), *sorted((ROOT / "hffn_amd").glob("*.py")), ROOT / "include" / "hffn_amd.h"]
    return Adapter(name="MI355X HIP leaf", load_pythia=pythia.load_pythia, device="cuda", synchronize=torch.cuda.synchronize,
                   state=_gpu_state, versions=_versions, describe=_runtime_report, runtime_files=sources,
                   note="one MI355X per box: ratios hold within one execution only")


# -- one cell, in its own process ---------------------------------------------------------------------------------------

@dataclass
class Cell:
    size: object
    density: int
    shape: str
    session: int = 0
    parity: int = 0
    blocks: int = 1
    window_ms: float = 60.0
    assets: str = ""

    def key(self) -> tuple:
        return self.size, self.density, self.shape


class ArmSet:
    """The three arms of one cell, their prompt and the dense arm's greedy continuation."""

    def __init__(self, adapter: Adapter, cell: Cell) -> None:
        from . import pythia
        self.adapter = adapter
        checkpoint, export = asset_dirs(Path(cell.assets), cell.size, cell.density)
        self.models = {arm: adapter.load_pythia(checkpoint, export, "hffn" if arm != "dense" else "dense", adapter.device)
                       for arm in ARMS}
        for arm in ("hffn", "hffn_copy"):
            pythia.share_non_ffn(self.models[arm], self.models["dense"])
        shape = SHAPES[cell.shape]
        vocab = self.models["dense"].config.vocab_size
        self.prompt = pythia.synthetic_prompts(shape["batch"], shape["prompt"], vocab).to(adapter.device)
        self.fed = self._greedy(shape["steps"])

    def _greedy(self, steps: int) -> list:
        """The dense arm's greedy tokens after the prompt, one [B, 1] tensor per decode step."""
        model, fed = self.models["dense"], []
        out = model(input_ids=self.prompt, use_cache=True)
        for _ in range(steps):
            fed.append(out.logits[:, -1:].argmax(-1))
            out = model(input_ids=fed[-1], past_key_values=out.past_key_values, use_cache=True)
        return fed

    def request(self, arm: str) -> list:
        """One request of ``arm`` (no synchronisation); the last-position logits of each of its calls."""
        model = self.models[arm]
        out = model(input_ids=self.prompt, use_cache=True)
        last = [out.logits[:, -1]]
        for token in self.fed:
            out = model(input_ids=token, past_key_values=out.past_key_values, use_cache=True)
            last.append(out.logits[:, -1])
        return last

    def window_ms(self, arm: str, repeats: int) -> float:
        """Milliseconds per request over ``repeats`` back-to-back requests between two synchronisations."""
        self.adapter.synchronize()
        began = time.perf_counter_ns()
        for _ in range(repeats):
            self.request(arm)
        self.adapter.synchronize()
        return (time.perf_counter_ns() - began) / repeats / 1e6


def gates(arms: ArmSet) -> dict:
    """The checks that precede any timing, from one request of each arm."""
    import torch
    seen = {arm: [logits.clone() for logits in arms.request(arm)] for arm in ARMS}
    same = all(bool(torch.equal(a, b)) for a, b in zip(seen["hffn"], seen["hffn_copy"]))
    largest = max(float(d.abs().max()) for d in seen["dense"])
    gap = max(float((h - d).abs().max()) for h, d in zip(seen["hffn"], seen["dense"])) / largest
    flips = sum(int((h.argmax(-1) != d.argmax(-1)).sum()) for h, d in zip(seen["hffn"], seen["dense"]))
    return {"bitwise_copy": same, "hffn_vs_dense_relative_gap": gap, "argmax_differing_positions": flips,
            "gate_passed": same and gap <= GUARD}


def block_order(parity: int, block: int) -> tuple[str, ...]:
    """The arms of one block: there and back, starting from the front or the back of ``ARMS``."""
    there = ARMS if (parity + block) % 2 == 0 else ARMS[::-1]
    return there + there[::-1]


def run_cell(adapter: Adapter, cell: Cell) -> dict:
    """Gates, then the timed windows of one cell; the row that the worker prints."""
    import torch
    with torch.inference_mode():
        arms = ArmSet(adapter, cell)
        row = {**{k: v for k, v in asdict(cell).items() if k != "assets"}, **gates(arms)}
        samples = {arm: [] for arm in ARMS}
        repeats = None
        if row["gate_passed"]:
            for arm in ARMS:
                arms.window_ms(arm, 2)  # buffers reserved, kernels and plans loaded
            single = min(arms.window_ms("dense", 1) for _ in range(3))
            repeats = max(1, min(MAX_REPEATS, int(cell.window_ms / single) + 1))
            for block in range(cell.blocks):
                for arm in block_order(cell.parity, block):
                    arms.window_ms(arm, repeats)  # untimed
                    samples[arm].append(arms.window_ms(arm, repeats))
        row.update(samples_ms=samples, repeats=repeats, runtime=adapter.describe(arms.models["hffn"]))
    return row


# -- many cells: the campaign -------------------------------------------------------------------------------------------

def aggregate(rows: list[dict]) -> list[dict]:
    """One entry per cell: median ms per arm over its sessions (each session's value the median of its windows), the
    hffn/dense ratios (median, min, max) and the A/A ratio of each session."""
    by_cell: dict = {}
    for row in rows:
        by_cell.setdefault((row["size"], row["density"], row["shape"]), []).append(
            {arm: statistics.median(row["samples_ms"][arm]) for arm in ARMS})
    cells = []
    for key in sorted(by_cell, key=lambda k: tuple(map(str, k))):
        sessions = by_cell[key]
        ratios = [s["hffn"] / s["dense"] for s in sessions]
        cells.append({"size": key[0], "density": key[1], "shape": key[2], "sessions": len(sessions),
                      "ms": {arm: statistics.median(s[arm] for s in sessions) for arm in ARMS},
                      "hffn_over_dense": statistics.median(ratios), "min": min(ratios), "max": max(ratios),
                      "aa": [s["hffn_copy"] / s["hffn"] for s in sessions]})
    return cells


def admissibility(cells: list[dict], complete: bool, gate_passed: bool) -> dict:
    """Whether the ratios may be read (criteria fixed before any measurement)."""
    if not complete:
        return {"admissible": False, "reason": "incomplete coverage"}
    aa = [ratio for cell in cells for ratio in cell["aa"]]
    within = [abs(ratio - 1.0) <= AA_TOLERANCE for ratio in aa]
    share = sum(within) / len(aa)
    return {"admissible": bool(gate_passed and share >= AA_SHARE), "gate_passed": gate_passed, "aa_values": len(aa),
            "aa_within_tolerance": sum(within), "aa_share": share, "aa_median": statistics.median(aa), "aa_min": min(aa),
            "aa_max": max(aa)}


def report(adapter_name: str, mode: str, done: int, planned: int, cells: list[dict], judged, failure) -> str:
    lines = [f"# Request-level harness, {adapter_name}, {mode}", "",
             f"{done} of {planned} processes completed ({'passed' if done == planned else 'failed'}).", "",
             "Milliseconds per request; read `hffn/dense` only when the verdict is admissible.", "",
             "| model | density | shape | dense | hffn | hffn/dense (min..max) | A/A by session |", "|---|---:|---|---:|---:|---|---|"]
    for c in cells:
        lines.append(f"| {c['size']}M | {c['density']} % | {c['shape']} | {c['ms']['dense']:.3f} | {c['ms']['hffn']:.3f} | "
                     f"{c['hffn_over_dense']:.3f} ({c['min']:.3f}..{c['max']:.3f}) | {' '.join(f'{a:.3f}' for a in c['aa'])} |")
    lines += ["", "Verdict:", "```json", json.dumps(judged, indent=1), "```"]
    if failure:
        lines += ["", "Stopped on:", "```", json.dumps(failure, indent=1)[:4000], "```"]
    return "\n".join(lines) + "\n"


def _sha256(path: Path) -> str:
    digest = hashlib.sha256()
    digest.update(Path(path).read_bytes())
    return digest.hexdigest()


def _subprocess_cell(cell: Cell) -> tuple[int, str, str]:
    done = subprocess.run([sys.executable, "-B", "-m", "hffn_amd.bench_request", "--worker", json.dumps(asdict(cell))],
                          text=True, capture_output=True, cwd=ROOT)
    return done.returncode, done.stdout, done.stderr


class Campaign:
    """Every (cell, session) of one grid in fresh processes; writes config.json, provenance.json, manifest.json,
    raw.jsonl, summary.json and REPORT.md into ``out``."""

    def __init__(self, adapter: Adapter, mode: str, assets: Path, out: Path, densities=None, sessions=None, sizes=None,
                 launcher=None) -> None:
        self.adapter, self.mode, self.assets, self.out = adapter, mode, Path(assets), Path(out)
        self.grid = dict(GRID[mode])
        for key, value in (("densities", densities), ("sessions", sessions), ("sizes", sizes)):
            if value:
                self.grid[key] = tuple(value) if key != "sessions" else value
        self.launcher = launcher or _subprocess_cell
        self.cells = [(s, d, shape) for s in self.grid["sizes"] for d in self.grid["densities"] for shape in self.grid["shapes"]]
        self.planned = len(self.cells) * self.grid["sessions"]
        self.manifest = {"status": "running", "planned": self.planned, "done": 0,
                         "started": datetime.now(timezone.utc).isoformat()}

    def _write(self, name: str, payload) -> None:
        text = payload if isinstance(payload, str) else json.dumps(payload, indent=1) + "\n"
        (self.out / name).write_text(text)

    def jobs(self):
        """(cell, its index in the grid) in run order: the grid forwards in even sessions, backwards in odd ones."""
        for session in range(self.grid["sessions"]):
            order = range(len(self.cells)) if session % 2 == 0 else range(len(self.cells) - 1, -1, -1)
            for index in order:
                size, density, shape = self.cells[index]
                yield Cell(size, density, shape, session=session, parity=(session + index) % 2, blocks=self.grid["blocks"],
                           window_ms=self.grid["window_ms"], assets=str(self.assets))

    def run(self) -> int:
        self.out.mkdir(parents=True, exist_ok=True)
        self._write("config.json", {"mode": self.mode, **self.grid, "arms": ARMS, "shape_definitions": SHAPES, "guard": GUARD,
                                    "aa_tolerance": AA_TOLERANCE, "aa_share": AA_SHARE})
        self._write("provenance.json", {"leaf": self.adapter.name, "versions": self.adapter.versions(),
                                        "runtime_files": {str(Path(p).relative_to(ROOT)): _sha256(p) for p in self.adapter.runtime_files},
                                        "state_at_start": self.adapter.state(), "machine": self.adapter.note})
        self._write("manifest.json", self.manifest)
        rows, failure = [], None
        with (self.out / "raw.jsonl").open("w") as raw:
            for cell in self.jobs():
                before = self.adapter.state()
                status, stdout, stderr = self.launcher(cell)
                printed = [line for line in stdout.splitlines() if line.startswith("{")]
                if status not in (0, GATE_FAILED) or not printed:
                    failure = {"cell": list(cell.key()), "session": cell.session, "returncode": status, "stderr": stderr[-4000:]}
                    break
                row = dict(json.loads(printed[-1]), state_before=before)
                raw.write(json.dumps(row) + "\n")
                raw.flush()
                rows.append(row)
                if status == GATE_FAILED:
                    failure = {"cell": list(cell.key()), "session": cell.session, "returncode": status,
                               "gates": {k: row.get(k) for k in ("bitwise_copy", "hffn_vs_dense_relative_gap", "gate_passed")}}
                    break
                self.manifest["done"] += 1
                self._write("manifest.json", self.manifest)
                medians = ", ".join(f"{arm} {statistics.median(row['samples_ms'][arm]):.3f}" for arm in ARMS)
                print(f"[{self.manifest['done']}/{self.planned}] session {cell.session} pythia{cell.size}m d{cell.density} "
                      f"{cell.shape} x{row['repeats']}: {medians} ms", flush=True)
        complete = self.manifest["done"] == self.planned
        gate_passed = failure is None or failure["returncode"] != GATE_FAILED
        cells = aggregate(rows) if complete else []
        judged = admissibility(cells, complete, gate_passed) if cells else None
        self._write("summary.json", {"cells": cells, "verdict": judged, "failure": failure, "state_at_end": self.adapter.state()})
        text = report(self.adapter.name, self.mode, self.manifest["done"], self.planned, cells, judged, failure)
        self._write("REPORT.md", text)
        self.manifest.update(status="passed" if complete else "failed", finished=datetime.now(timezone.utc).isoformat())
        self._write("manifest.json", self.manifest)
        print(text, flush=True)
        return 0 if complete else 1


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--worker", help="one cell (JSON) in this process")
    parser.add_argument("--mode", choices=sorted(GRID))
    parser.add_argument("--assets", type=Path, help="holds pythia<size>m/ checkpoints and pythia<size>m_sparse<d>/export/")
    parser.add_argument("--prepare", action="store_true", help="write the missing random-init checkpoints and exports first")
    parser.add_argument("--out", type=Path)
    parser.add_argument("--densities", type=lambda text: tuple(int(v) for v in text.split(",")))
    parser.add_argument("--sessions", type=int)
    parser.add_argument("--sizes", type=lambda text: tuple(int(v) for v in text.split(",")))
    args = parser.parse_args(argv)
    adapter = hip_adapter()
    if args.worker:
        row = run_cell(adapter, Cell(**json.loads(args.worker)))
        print(json.dumps(row), flush=True)
        return 0 if row["gate_passed"] else GATE_FAILED
    if not (args.mode and args.assets and args.out):
        parser.error("--mode, --assets and --out are required")
    sizes = args.sizes or GRID[args.mode]["sizes"]
    densities = args.densities or GRID[args.mode]["densities"]
    if args.prepare:
        for folder in prepare(args.assets, {s: SIZES[s] for s in sizes}, densities):
            print(f"wrote {folder}", flush=True)
    missing = [str(path) for s in sizes for d in densities
               for path in (asset_dirs(args.assets, s, d)[0] / "model.safetensors", asset_dirs(args.assets, s, d)[1] / "layer0")
               if not path.exists()]
    if missing:
        raise SystemExit(f"missing assets (use --prepare): {missing}")
    return Campaign(adapter, args.mode, args.assets, args.out, args.densities, args.sessions, args.sizes).run()


if __name__ == "__main__":
    sys.exit(main())
