#!/usr/bin/env python3
"""HFFN layer throughput on one MI355X: tokens/s of the isolated layer and the roofline fraction of its dominant kernel.

Workload (default): the Pythia-410M-shape HFFN layer, d_model 1024, d_ff 4096, 50 % density (512-slot up and down
supports per neuron, uniform without replacement, sorted), fp32 values ~N(0, 0.02), biases ~N(0, 0.01), x = 2048 tokens
~N(0, 1), exact-erf GELU. A step is one forward of the whole layer on the 2048 resident tokens. The timed loop rotates
over enough copies of the layer (device clones of its arrays, each at its own addresses) that their stores exceed the
256 MB Infinity Cache, so every step reads its model from HBM.

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
    parser.add_argument("--settle-ms", type=float, default=500.0,
                        help="after the warm-up steps, untimed rotations over the copies for this long (GPU clocks ramp "
                             "up under load: 20 steps after 5 warm-up steps measured 0.141 ms per step, 200 after 20 "
                             "0.122 ms)")
    parser.add_argument("--no-decode", action="store_true", help="skip the decode record")
    parser.add_argument("--tiled", action="store_true",
                        help="the runtime with tiled copies of the stores (tiled=True: the tiles path reads interleaved "
                             "copies instead of the compact rows)")
    parser.add_argument("--decode-rotations", type=int, default=20, help="passes over the copies per decode entry")
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


def _kernel_seconds(recorded: list, names: list[str], steps: int) -> dict:
    torch.cuda.synchronize()
    return {name: sum(e[i].elapsed_time(e[i + 1]) for e in recorded) * 1e-3 / steps for i, name in enumerate(names)}


def time_kernels(runtime, x: torch.Tensor, steps: int, copies: int) -> dict:
    """Average duration (s) of each kernel of the step, from HIP events recorded between the launches on the
    current stream (the stream the C ABI launches on); the steps are issued back to back, without a synchronisation
    between them, so that no launch latency of an idle device enters the figures."""
    from hffn_amd import _lib
    from hffn_amd.runtime import leading_dim

    lib = _lib.load()
    n = x.shape[0]
    ld = leading_dim(n)
    up, down = runtime.modes(n)
    x_t, act, y_t, y = runtime._work
    stream = torch.cuda.current_stream().cuda_stream
    recorded = []  # the steps run back to back; the events are read after the last one
    if up == "mfma":
        # hffn_mfma_up's two halves apart (the input split, then the up GEMM), so that the GEMM is priced alone
        names = ["split", "up", "down"]
        work, work_bytes = runtime._mfma_work.data_ptr(), 4 * runtime._mfma_work.numel()
        for step in range(steps):
            index = step % copies
            value_type = runtime._args[index][0]
            planes, tensors = runtime._planes[index], runtime._tensors[index]
            events = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
            events[0].record()
            _lib.check(lib.hffn_mfma_split(x.data_ptr(), work, work_bytes, runtime.d_model, runtime.d_ff, n, stream), "mfma split")
            events[1].record()
            _lib.check(lib.hffn_mfma_up_planes(value_type, planes["up"].data_ptr(), planes["up_binades"].data_ptr(),
                                               tensors["b_up"].data_ptr(), work, work_bytes, runtime.d_model, runtime.d_ff, n,
                                               stream), "mfma up")
            events[2].record()
            _lib.check(lib.hffn_mfma_down(value_type, planes["down"].data_ptr(), planes["down_binades"].data_ptr(),
                                          tensors["b_down"].data_ptr(), y, work, work_bytes, runtime.d_model, runtime.d_ff, n, stream),
                       "mfma down")
            events[3].record()
            recorded.append(events)
        return _kernel_seconds(recorded, names, steps)
    if up in ("gemv", "tiles"):  # both projections in one ABI call, timed as one
        work, work_bytes = runtime._gemv_work.data_ptr(), 4 * runtime._gemv_work.numel()
        for step in range(steps):
            index = step % copies
            value_type = runtime._args[index][0]
            events = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            events[0].record()
            if up == "tiles":
                runtime._tiles_forward(index, x, n, stream)
            else:
                planes, tensors = runtime._planes[index], runtime._tensors[index]
                _lib.check(lib.hffn_forward_gemv(value_type, x.data_ptr(), planes["up"].data_ptr(), planes["up_binades"].data_ptr(),
                                                 tensors["b_up"].data_ptr(), planes["down"].data_ptr(),
                                                 planes["down_binades"].data_ptr(), tensors["b_down"].data_ptr(), act, work,
                                                 work_bytes, y, runtime.d_model, runtime.d_ff, n, stream), "gemv")
            events[1].record()
            recorded.append(events)
        return _kernel_seconds(recorded, [up], steps)
    names = (["transpose_in"] if up == "rows" else []) + ["up", "down"] + (["transpose_out"] if down == "rows" else [])
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
        recorded.append(events)
    return _kernel_seconds(recorded, names, steps)


DECODE_TOKENS = {"pythia410m_d50": (1, 8, 16), "pythia1p4b_d20_bf16": (1, 4, 16)}
DECODE_STEP_BATCHES = (1, 8)
DECODE_STEP_LAYERS = 24


def device_copies(layer, count: int) -> list:
    """``layer`` and count - 1 clones of its device arrays: the same store at distinct addresses, so that a rotation
    over them reads HBM on every call as distinct layers would (the timing does not depend on the values)."""
    from hffn_amd.runtime import HFFNLayer
    return [layer] + [HFFNLayer(**{k: v.clone() if isinstance(v, torch.Tensor) else v for k, v in vars(layer).items()})
                      for _ in range(count - 1)]


def call_us(runtime, x: torch.Tensor, copies: int, rotations: int) -> float:
    """Mean µs of one ``forward`` over ``rotations`` passes through the copies (HIP events around all of them), after
    one untimed pass (inputs resident)."""
    for index in range(copies):
        runtime.forward(index, x)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(rotations):
        for index in range(copies):
            runtime.forward(index, x)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / (rotations * copies)


def read_floor(compact, copies: int, rotations: int, device) -> dict:
    """The plain-read floor of a decode call (``hffn_read_probe``): the bytes of the layer's up and down stores (offsets,
    slots, bias) read by a kernel that does nothing else, from ``copies`` distinct buffers in rotation, as one launch
    per side back to back (the call's two dependent kernels) and as one launch for both; µs per call, events around
    ``rotations`` passes after one untimed pass."""
    from hffn_amd import _lib
    lib = _lib.load()
    costs = layer_costs(compact, 1)
    sides = [costs["up"]["bytes"] - 4 * (compact.d_model + compact.d_ff), costs["down"]["bytes"] - 4 * (compact.d_model + compact.d_ff)]
    sides = [(b + 15) // 16 * 16 for b in sides]
    buffers = [torch.empty(sum(sides), dtype=torch.uint8, device=device) for _ in range(copies)]
    blocks = lambda size: min(8192, max(256, size // 12288))  # ~3 KB per wave  # noqa: E731
    sink = torch.empty(4 * blocks(sum(sides)), dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream

    def read(pointer: int, size: int) -> None:
        _lib.check(lib.hffn_read_probe(pointer, size, sink.data_ptr(), sink.numel(), blocks(size), stream), "read probe")

    def timed(one_launch: bool) -> float:
        def run(buffer):
            if one_launch:
                read(buffer.data_ptr(), sum(sides))
            else:
                read(buffer.data_ptr(), sides[0])
                read(buffer.data_ptr() + sides[0], sides[1])
        for buffer in buffers:
            run(buffer)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(rotations):
            for buffer in buffers:
                run(buffer)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e3 / (rotations * copies)

    two, one = timed(False), timed(True)
    del buffers
    return {"bytes_per_side": sides, "two_launches_us": round(two, 2), "one_launch_us": round(one, 2),
            "two_launches_hbm_fraction": round(sum(sides) / (two * 1e-6) / HBM_PEAK, 4),
            "one_launch_hbm_fraction": round(sum(sides) / (one * 1e-6) / HBM_PEAK, 4)}


def decode_entry(runtime, workload, compact, n: int, copies: int, rotations: int, device, floor: dict | None = None) -> dict:
    from hffn_amd import synth
    x = torch.from_numpy(synth.make_input(workload, n)).to(device)
    us = call_us(runtime, x, copies, rotations)
    moved = layer_costs(compact, n)["step_bytes"]  # the compact store, x read, y written
    entry = {"tokens": n, "modes": list(runtime.modes(n)), "us_per_call": round(us, 2), "tokens_per_s": round(n / us * 1e6, 1),
             "hbm_fraction": round(moved / (us * 1e-6) / HBM_PEAK, 4)}
    if floor:  # the call's time against a plain read of its stores in two launches
        entry["of_read_floor"] = round(floor["two_launches_us"] / us, 3)
    return entry


def decode_record(runtime, base, device, rotations: int, steps: int) -> dict:
    """Decode-sized calls in the same process after the headline: the Pythia-410M-shape layer (the headline's copies)
    at 1, 8 and 16 tokens; the Pythia-1.4B-shape bf16 layer at 20 % at 1, 4 and 16 tokens (one generated layer and
    device clones, more than 300 MB in the rotation); and the FFN calls of one decode step of the 24-layer
    Pythia-410M-shape model at batch 1 and 8, eager and replayed from a HIP graph (hffn_amd.bench_decode). Every
    entry: µs per call (or step), the HBM fraction on the compact bytes it reads, and the fraction of the plain-read
    floor (``read_floor``: the same bytes read by a kernel that does nothing else, one launch per side)."""
    from hffn_amd import bench_decode, synth
    from hffn_amd.ffn import hip_layer
    from hffn_amd.prepared_runtime import PreparedRuntime
    from hffn_amd.runtime import HFFNRuntime

    record = {"rotation": f"{rotations} passes over each layer's copies after one untimed pass; HIP events around all",
              "tiled": runtime.tiled}
    w410 = synth.WORKLOADS["pythia410m_d50"]
    if (runtime.d_model, runtime.d_ff) != (w410.d_model, w410.d_ff):  # another headline layer: the 410M layer of its own
        base = synth.make_workload_layer(w410)
        count = max(1, math.ceil(MALL_BYTES / layer_costs(base, 1)["model_bytes"]))
        runtime = HFFNRuntime(device_copies(hip_layer(base, device), count), device, tiled=runtime.tiled)
    copies = len(runtime.layers)
    floor = read_floor(base, copies, rotations, device)
    record["pythia410m_d50_read_floor"] = floor
    record["pythia410m_d50"] = [decode_entry(runtime, synth.WORKLOADS["pythia410m_d50"], base, n, copies, rotations, device, floor)
                                for n in DECODE_TOKENS["pythia410m_d50"]]
    workload = synth.WORKLOADS["pythia1p4b_d20_bf16"]
    compact = synth.make_workload_layer(workload)
    count = max(1, math.ceil(MALL_BYTES / layer_costs(compact, 1)["model_bytes"]))
    bf16 = HFFNRuntime(device_copies(hip_layer(compact, device), count), device, tiled=runtime.tiled)
    bf16_floor = read_floor(compact, count, rotations, device)
    record["pythia1p4b_d20_bf16_read_floor"] = bf16_floor
    record["pythia1p4b_d20_bf16"] = [decode_entry(bf16, workload, compact, n, count, rotations, device, bf16_floor)
                                     for n in DECODE_TOKENS["pythia1p4b_d20_bf16"]]
    del bf16
    layers = runtime.layers + device_copies(runtime.layers[0], DECODE_STEP_LAYERS - copies + 1)[1:]
    model = PreparedRuntime(layers[:DECODE_STEP_LAYERS], device, tiled=runtime.tiled)
    record["pythia410m_model_step"] = [bench_decode.measure(model, [base] * DECODE_STEP_LAYERS, batch, steps)
                                       for batch in DECODE_STEP_BATCHES]
    for entry in record["pythia410m_model_step"]:  # against the plain read of every layer's stores, two launches each
        entry["of_read_floor"] = round(DECODE_STEP_LAYERS * floor["two_launches_us"] / entry["calls_us_per_step"], 3)
    del model
    torch.cuda.empty_cache()
    return record


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
    runtime = HFFNRuntime(device_copies(hip_layer(base, device), copies), device, tiled=args.tiled)
    x_np = synth.make_input(workload, n)
    x = torch.from_numpy(x_np).to(device)

    for step in range(args.warmup):
        runtime.forward(step % copies, x)
    for index in range(copies):  # every copy once, untimed: none is first used inside the timed steps
        runtime.forward(index, x)
    torch.cuda.synchronize()
    settle = time.perf_counter()
    while time.perf_counter() - settle < args.settle_ms * 1e-3:  # untimed rotations until the clocks have ramped up
        for index in range(copies):
            runtime.forward(index, x)
        torch.cuda.synchronize()
    settle = time.perf_counter() - settle
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
    decode = None if args.no_decode else decode_record(runtime, base, device, args.decode_rotations, 50)
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
                   "warmup_rotation": "after the warm-up steps, every copy called once untimed, then untimed "
                                      f"rotations for {settle:.2f} s (clock ramp)",
                   "modes": [up, down], "kernel_us": {k: round(v * 1e6, 2) for k, v in kernels.items()},
                   "step_hbm_fraction": round(costs["step_bytes"] / (seconds / args.steps) / HBM_PEAK, 4),
                   "step_fp32_fraction": round(costs["step_flops"] / (seconds / args.steps) / FP32_PEAK, 4),
                   "memory_bytes": {"compact_store": costs["model_bytes"], "planes": runtime.dense_bytes() // copies,
                                    ("tiled_store" if runtime.tiled else "row_bounds_tables"): runtime.tiles_bytes() // copies,
                                    "workspace": runtime.workspace_bytes()},
                   "tiled": runtime.tiled,
                   "wall_s": round(wall, 3)},
        "roofline": roofline,
        "cpu_baseline": baseline,
        "decode": decode,
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
