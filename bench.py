#!/usr/bin/env python3
"""HFFN layer throughput on one MI355X: tokens/s of the isolated layer and the roofline fraction of its dominant kernel.

Workload (default): the Pythia-410M-shape HFFN layer, d_model 1024, d_ff 4096, 50 % density (512-slot up and down
supports per neuron, uniform without replacement, sorted), fp32 values ~N(0, 0.02), biases ~N(0, 0.01), x = 2048 tokens
~N(0, 1), exact-erf GELU. A step is one forward of the whole layer on the 2048 resident tokens. The timed loop rotates
over enough distinct copies of the layer (different seeds) that their stores exceed the 256 MB Infinity Cache, so
every step reads its model from HBM.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--tokens N]

Prints one JSON line. `roofline` is measured live: HIP events around each kernel of the step (on the stream the
kernels are launched on) give each kernel's average duration; the dominant one is priced against its algorithmic
bytes or flops: the tile-densified MFMA path against the dense fp16 MFMA peak times the side's useful/dense flop ratio
(with the fp32-equivalent fraction and the issued fp16 MFMA rate beside it), the gather kernels at large N against the
fp32 peak, decode-sized calls against HBM on the compact store's bytes (the decode GEMVs also on the bytes of the planes
they read). `traffic` comes from the committed rocprofv3 counter summary of the same command. `cpu_baseline` times the
reference x86 AVX2 kernel (built from the reference source into oracle/_ref) on this host's cores, pinned, in child
processes started before this process touches the GPU (oracle.cpu_bench: the bench workload and the 70M-shape CPU
configuration, at 8 threads and at every physical core of one NUMA node within the host's CPU share).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402
import torch  # noqa: E402

METRIC = "HFFN layer tokens/s + % HBM roofline, Pythia-410M shape @50% density"
HBM_PEAK = 8.0e12          # bytes/s, MI355X HBM3E
FP32_PEAK = 157.3e12       # FLOP/s, MI355X fp32 (vector and matrix)
FP16_MFMA_PEAK = 2.5e15    # FLOP/s, MI355X dense fp16 MFMA
RIDGE = FP32_PEAK / HBM_PEAK
MALL_BYTES = 300e6         # rotate over more than the 256 MB Infinity Cache


def parse() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--workload", default="pythia410m_d50")
    parser.add_argument("--tokens", type=int, default=None, help="N (default: the workload's first token count)")
    parser.add_argument("--copies", type=int, default=None, help="distinct layer copies in the rotation")
    parser.add_argument("--cpu-seconds", type=float, default=5.0, help="timed seconds per CPU-baseline run (4 runs)")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--copy-probe-mb", type=int, default=0,
                        help="after the run, copy a buffer of this many MiB 3 times (the plain copy kernel that "
                             "calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return parser.parse_args()


TRAFFIC = ROOT / "profiles" / "traffic.json"


def measured_traffic(workload: str, n: int, kernel: str) -> int | None:
    """Memory-side bytes per launch of `kernel` ("up (mfma)", ...), from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary of this workload (each counter scaled by its copy-kernel calibration), or None when none matches."""
    if not TRAFFIC.exists():
        return None
    record = json.loads(TRAFFIC.read_text()).get("workloads", {}).get(f"{workload}/n{n}", {}).get(kernel)
    return int(record["traffic_bytes"]) if record else None


def layer_costs(compact, n: int) -> dict:
    """Algorithmic bytes and flops of each kernel of one step (model arrays read once, activations once)."""
    d, h = compact.d_model, compact.d_ff
    value = 2 if compact.value_dtype == "bf16" else 4
    nnz_up, nnz_down = int(compact.up_idx.size), int(compact.down_idx.size)
    up_store = 4 * (h + 1) + (2 + value) * nnz_up + 4 * h
    down_store = 4 * (d + 1) + (2 + value) * nnz_down + 4 * d
    return {
        "transpose_in": {"bytes": 8 * n * d, "flops": 0},
        "up": {"bytes": up_store + 4 * n * d + 4 * n * h, "flops": 2 * nnz_up * n},
        "down": {"bytes": down_store + 4 * n * h + 4 * n * d, "flops": 2 * nnz_down * n},
        "transpose_out": {"bytes": 8 * n * d, "flops": 0},
        # the decode GEMVs run both projections in one ABI call (timed as one); priced on the same algorithmic bytes
        "gemv": {"bytes": up_store + down_store + 8 * n * d + 8 * n * h, "flops": 2 * (nnz_up + nnz_down) * n},
        "model_bytes": up_store + down_store,
        "step_bytes": up_store + down_store + 8 * n * d,
        "step_flops": 2 * (nnz_up + nnz_down) * n,
        "density_up": nnz_up / (d * h), "density_down": nnz_down / (d * h), "density": (nnz_up + nnz_down) / (2 * d * h),
    }


def time_kernels(runtime, x: torch.Tensor, steps: int, copies: int) -> dict:
    """Average duration (s) of each kernel of the step, from HIP events recorded between the launches on the
    current stream (the stream the C ABI launches on)."""
    from hffn_amd import _lib
    from hffn_amd.runtime import leading_dim

    lib = _lib.load()
    n = x.shape[0]
    ld = leading_dim(n)
    up, down = runtime.modes(n)
    x_t, act, y_t, y = runtime._work
    stream = torch.cuda.current_stream().cuda_stream
    if up == "mfma":
        names = ["up", "down"]
        totals = {name: 0.0 for name in names}
        work, work_bytes = runtime._mfma_work.data_ptr(), 4 * runtime._mfma_work.numel()
        for step in range(steps):
            index = step % copies
            value_type = runtime._args[index][0]
            planes, tensors = runtime._planes[index], runtime._tensors[index]
            events = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
            events[0].record()
            _lib.check(lib.hffn_mfma_up(value_type, x.data_ptr(), planes["up"].data_ptr(), planes["up_binades"].data_ptr(),
                                        tensors["b_up"].data_ptr(), work, work_bytes, runtime.d_model, runtime.d_ff, n, stream),
                       "mfma up")
            events[1].record()
            _lib.check(lib.hffn_mfma_down(value_type, planes["down"].data_ptr(), planes["down_binades"].data_ptr(),
                                          tensors["b_down"].data_ptr(), y, work, work_bytes, runtime.d_model, runtime.d_ff, n, stream),
                       "mfma down")
            events[2].record()
            torch.cuda.synchronize()
            for i, name in enumerate(names):
                totals[name] += events[i].elapsed_time(events[i + 1]) * 1e-3
        return {name: total / steps for name, total in totals.items()}
    if up in ("gemv", "tiles"):  # both projections in one ABI call, timed as one
        total = 0.0
        work, work_bytes = runtime._gemv_work.data_ptr(), 4 * runtime._gemv_work.numel()
        for step in range(steps):
            index = step % copies
            value_type = runtime._args[index][0]
            events = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            events[0].record()
            if up == "tiles":
                _lib.check(lib.hffn_forward_tiles(value_type, x.data_ptr(), *runtime._tiles_args(index), runtime.d_model,
                                                  runtime.d_ff, *runtime._nnz[index], n, stream), "tiles")
            else:
                planes, tensors = runtime._planes[index], runtime._tensors[index]
                _lib.check(lib.hffn_forward_gemv(value_type, x.data_ptr(), planes["up"].data_ptr(), planes["up_binades"].data_ptr(),
                                                 tensors["b_up"].data_ptr(), planes["down"].data_ptr(),
                                                 planes["down_binades"].data_ptr(), tensors["b_down"].data_ptr(), act, work,
                                                 work_bytes, y, runtime.d_model, runtime.d_ff, n, stream), "gemv")
            events[1].record()
            torch.cuda.synchronize()
            total += events[0].elapsed_time(events[1]) * 1e-3
        return {up: total / steps}
    names = (["transpose_in"] if up == "rows" else []) + ["up", "down"] + (["transpose_out"] if down == "rows" else [])
    totals = {name: 0.0 for name in names}
    for step in range(steps):
        value_type, up_off, up_idx, up_val, b_up, out_off, out_hid, out_val, b_down = runtime._args[step % copies]
        nnz_up, nnz_down = runtime._nnz[step % copies]
        events = [torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
        events[0].record()
        k = 1
        if up == "rows":
            _lib.check(lib.hffn_transpose(x.data_ptr(), x_t, n, runtime.d_model, runtime.d_model, ld, stream), "transpose")
            events[k].record(); k += 1
            _lib.check(lib.hffn_up(_lib.UP_MODES[up], value_type, x_t, up_off, up_idx, up_val, b_up, act, runtime.d_model,
                                   runtime.d_ff, nnz_up, n, ld, stream), "up")
        else:
            _lib.check(lib.hffn_up(_lib.UP_MODES[up], value_type, x.data_ptr(), up_off, up_idx, up_val, b_up, act,
                                   runtime.d_model, runtime.d_ff, nnz_up, n, ld, stream), "up")
        events[k].record(); k += 1
        target = y_t if down == "rows" else y
        _lib.check(lib.hffn_down(_lib.DOWN_MODES[down], value_type, act, out_off, out_hid, out_val, b_down, target,
                                 runtime.d_model, runtime.d_ff, nnz_down, n, ld, stream), "down")
        events[k].record(); k += 1
        if down == "rows":
            _lib.check(lib.hffn_transpose(y_t, y, runtime.d_model, n, ld, runtime.d_model, stream), "transpose")
            events[k].record(); k += 1
        torch.cuda.synchronize()
        for i, name in enumerate(names):
            totals[name] += events[i].elapsed_time(events[i + 1]) * 1e-3
    return {name: total / steps for name, total in totals.items()}


def _child_json(arguments: list[str]) -> dict:
    """One pinned child process of oracle.cpu_bench (started before this process touches the GPU); its JSON line."""
    import subprocess
    done = subprocess.run([sys.executable, "-m", "oracle.cpu_bench", *arguments], cwd=ROOT, text=True, capture_output=True,
                          timeout=600)
    lines = [line for line in done.stdout.splitlines() if line.startswith("{")]
    if done.returncode != 0 or not lines:
        raise RuntimeError(f"oracle.cpu_bench {' '.join(arguments)} failed ({done.returncode}): {done.stderr[-2000:]}")
    return json.loads(lines[-1])


def cpu_baseline(workload: str, n: int, seconds: float) -> dict | None:
    """The reference x86 kernel on this host, pinned (oracle.cpu_bench, the protocol of the reference's
    bench/threads.py): the bench workload and the 70M-shape CPU configuration (128 tokens), each at T = 8 and at
    T = every physical core of NUMA node 0 that this process may use (at most 64, and at most the host CPU share
    OMP_NUM_THREADS names when set). ``value`` is the faster of the two runs of the bench workload, by wall time."""
    from oracle import cpu_bench, x86_ref

    if not x86_ref.available():
        return None
    host = cpu_bench.machine()
    node = next(iter(host["numa"].values()), {"cpus": host["affinity"]})
    cores = cpu_bench.one_core_per_node_cpu(node["cpus"], set(host["affinity"])) or host["affinity"]
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    every = cores[:min(64, len(cores), share or len(cores))]
    settings = [("T8", cores[:8]), ("T_all", every)] if len(every) > 8 else [("T8", cores[:8])]
    runs = []
    for name, cpus in settings:
        for wl, tokens, budget in ((workload, n, seconds), ("pythia70m_d20", 128, min(seconds, 4.0))):
            row = _child_json(["--cpus", ",".join(map(str, cpus)), "--threads", str(len(cpus)), "--workload", wl,
                               "--tokens", str(tokens), "--seconds", str(budget)])
            runs.append({"setting": name, **{k: row[k] for k in ("workload", "tokens", "threads", "calls", "kernel_us_median",
                                                               "wall_us_median", "tokens_per_s_wall", "tokens_per_s_kernel",
                                                               "max_abs_error_vs_float64")}})
    main_runs = [r for r in runs if r["workload"] == workload]
    best = max(main_runs, key=lambda r: r["tokens_per_s_wall"])
    return {"value": best["tokens_per_s_wall"], "unit": "tokens/s", "cores": best["threads"], "kind": "reference",
            "sample": f"{best['calls']} whole {n}-token calls of the same layer, median wall "
                      f"{best['wall_us_median'] / 1e3:.2f} ms (in-kernel {best['kernel_us_median'] / 1e3:.2f} ms), "
                      f"process pinned to {best['threads']} cores of NUMA node 0, {best['threads']} threads, route dual in "
                      f"96-token chunks; checked against the float64 oracle on 96 tokens",
            "runs": runs, "machine": {k: host[k] for k in ("model", "logical_cpus", "governor")} |
            {"numa_nodes": len(host["numa"]), "node0_physical_cores": node.get("physical_cores"), "allowed_cpus": len(host["affinity"])}}


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the HFFN layer runs on a single MI355X here (multi-GPU sharding is design "
              "only); run it with --gpus 1", file=sys.stderr)
        return 2
    from hffn_amd import synth
    from hffn_amd.ffn import hip_layer
    from hffn_amd.runtime import HFFNRuntime

    workload = synth.WORKLOADS[args.workload]
    n = args.tokens or workload.tokens[0]
    # the CPU baseline first, in pinned child processes, while this process has not touched the GPU
    baseline = None if args.no_cpu else cpu_baseline(workload.name, n, args.cpu_seconds)
    device = torch.device("cuda", 0)
    base = synth.make_workload_layer(workload)
    costs = layer_costs(base, n)
    copies = args.copies or max(1, math.ceil(MALL_BYTES / costs["model_bytes"]))
    compacts = [base] + [synth.make_workload_layer(workload, seed=workload.seed * 1000 + c) for c in range(1, copies)]
    runtime = HFFNRuntime([hip_layer(c, device) for c in compacts], device)
    x_np = synth.make_input(workload, n)
    x = torch.from_numpy(x_np).to(device)

    for step in range(args.warmup):
        runtime.forward(step % copies, x)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall = time.perf_counter()
    start.record()
    for step in range(args.steps):
        runtime.forward(step % copies, x)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall
    seconds = start.elapsed_time(end) * 1e-3
    up, down = runtime.modes(n)

    kernels = time_kernels(runtime, x, max(20, min(args.steps, 200)), copies)
    dominant = max((k for k in kernels if k in ("up", "down", "gemv", "tiles")), key=kernels.get)
    cost = costs["gemv" if dominant == "tiles" else dominant]
    seconds_kernel = kernels[dominant]
    density = {"up": costs["density_up"], "down": costs["density_down"]}.get(dominant, costs["density"])
    if up == "mfma" and dominant in ("up", "down"):
        # The tile-densified MFMA path: its useful flops against the dense fp16 MFMA peak scaled by the useful/dense
        # flop ratio of the side (its support density); beside it, the same flops against the fp32 peak, and what the
        # MFMA units issue (the dense products of the planes: 3 fp16 MFMAs per product for fp32 values, 2 for bf16).
        achieved = cost["flops"] / seconds_kernel
        peak = FP16_MFMA_PEAK * density
        products = 2 if base.value_dtype == "bf16" else 3
        roofline = {"bound": "mfma", "achieved": round(achieved / 1e12, 3), "peak": round(peak / 1e12, 1), "unit": "TFLOP/s",
                    "frac": round(achieved / peak, 4),
                    "peak_rule": "dense fp16 MFMA 2.5 PFLOP/s x useful/dense flops (the side's support density)",
                    "fp32_equivalent_frac": round(achieved / FP32_PEAK, 4),
                    "fp16_mfma_issued_frac": round(2 * n * base.d_model * base.d_ff * products / seconds_kernel / FP16_MFMA_PEAK, 4)}
    elif cost["flops"] / cost["bytes"] > RIDGE:  # the gather kernels at large N: fp32 FMAs
        achieved = cost["flops"] / seconds_kernel
        roofline = {"bound": "mfma", "achieved": round(achieved / 1e12, 3), "peak": FP32_PEAK / 1e12, "unit": "TFLOP/s",
                    "frac": round(achieved / FP32_PEAK, 4), "peak_rule": "fp32 157.3 TFLOP/s (vector FMAs)"}
    else:
        achieved = cost["bytes"] / seconds_kernel
        roofline = {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK, 4), "peak_rule": "HBM3E 8 TB/s on the compact store's bytes"}
        if dominant == "gemv":  # what the decode GEMVs read: the densified planes instead of the compact store
            # bf16 weights are read from the hi plane only: half of the bytes the planes occupy
            held = runtime.dense_bytes() // copies // (2 if base.value_dtype == "bf16" else 1)
            planes = held + costs["step_bytes"] - costs["model_bytes"]
            roofline["planes_bytes"] = int(planes)
            roofline["frac_on_planes_bytes"] = round(planes / seconds_kernel / HBM_PEAK, 4)
    names = {"gemv": "up+down (gemv)", "tiles": "up+down (tiles)"}
    roofline["kernel"] = names.get(dominant, f"{dominant} ({up if dominant == 'up' else down})")
    roofline["traffic"] = measured_traffic(workload.name, n, roofline["kernel"])
    roofline["traffic_source"] = ("rocprofv3 FETCH_SIZE + WRITE_SIZE of this command, per launch, scaled by the copy-kernel "
                                  "calibration: profiles/traffic.json" if roofline["traffic"] is not None else None)
    roofline["kernel_us"] = round(seconds_kernel * 1e6, 2)

    line = {
        "metric": METRIC, "value": round(n * args.steps / seconds, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(seconds / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32" if base.value_dtype == "float32" else "bf16-weights/f32-accumulate", "data": "synthetic",
        "config": {"workload": f"{workload.name}: isolated HFFN layer d_model={base.d_model} d_ff={base.d_ff}, "
                               f"{workload.degree}-slot supports, {n} tokens", "tokens": n, "copies": copies,
                   "modes": [up, down], "kernel_us": {k: round(v * 1e6, 2) for k, v in kernels.items()},
                   "step_hbm_fraction": round(costs["step_bytes"] / (seconds / args.steps) / HBM_PEAK, 4),
                   "step_fp32_fraction": round(costs["step_flops"] / (seconds / args.steps) / FP32_PEAK, 4),
                   "memory_bytes": {"compact_store": costs["model_bytes"], "planes": runtime.dense_bytes() // copies,
                                    "tiled_store": runtime.tiles_bytes() // copies, "workspace": runtime.workspace_bytes()},
                   "wall_s": round(wall, 3)},
        "roofline": roofline,
        "cpu_baseline": baseline,
    }
    print(json.dumps(line), flush=True)
    if args.copy_probe_mb:
        source = torch.empty(args.copy_probe_mb << 18, device=device)
        target = torch.empty_like(source)
        for _ in range(3):
            target.copy_(source)
        torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
