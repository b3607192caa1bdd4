"""FFN time of one decode step of a Pythia-410M-shape model on one GPU: the 24 FFN calls of a step that advances a batch
of B sequences by one token (B tokens per call), each layer d_model 1024, d_ff 4096, 512-slot supports (50 %), float32
weights, against the HBM roofline on the 24 layers' compact-store bytes (FFN bytes per step over FFN time). No
reference counterpart: the reference times whole requests, prompt plus cached decode steps, with every model part
(``runtime/gpu/nvidia/llm/inference/bench/bench_request.py``; here ``hffn_amd.bench_request``).

    python -m hffn_amd.bench_decode [--batch 1,8,16] [--steps 50] [--layers 24]

Two ways of issuing a step: eager (24 ``PreparedRuntime.forward`` calls, each launched from its plan) and replayed
from a HIP graph of the same 24 calls captured once per batch size (PyTorch's ``torch.cuda.CUDAGraph`` around the
calls on the capture stream; the library's launches carry no allocation, copy, memset or synchronisation). The FFN
time is that of the calls alone (``calls_*``: each output stays in the runtime's buffer, as a model's residual sum
reads it there); beside it, the step with each output copied out of the buffer (``with_copies_*``: one more PyTorch
kernel per layer), whose graph replays are checked bit for bit against the eager step's, with eager work between
replays. One JSON line per batch size: microseconds per step (HIP events around ``steps`` steps after warm-up, inputs
resident), per layer, and the HBM fraction of the faster way on the compact bytes. The layers are synthetic
(``synth``), one per model layer.
"""
from __future__ import annotations

import argparse
import json

import torch

from . import synth
from .ffn import hip_layer
from .prepared_runtime import PreparedRuntime

HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s
WORKLOAD = synth.WORKLOADS["pythia410m_d50"]


def compact_bytes(layer: synth.CompactLayer) -> int:
    """Bytes of the compact store one call reads: offsets, the slots of both sides (int16 index + value), biases."""
    value = 2 if layer.value_dtype == "bf16" else 4
    return (4 * (layer.d_ff + 1) + (2 + value) * layer.up_idx.size + 4 * layer.d_ff
            + 4 * (layer.d_model + 1) + (2 + value) * layer.down_idx.size + 4 * layer.d_model)


def step(runtime: PreparedRuntime, xs: list[torch.Tensor], outs: list[torch.Tensor]) -> None:
    """One decode step's FFN calls: layer i on xs[i] (the layers do not feed each other here: the attention and
    residual work between them is not part of the FFN time), each output copied out of the runtime's buffer."""
    for i, x in enumerate(xs):
        outs[i].copy_(runtime.forward(i, x))


def calls(runtime: PreparedRuntime, xs: list[torch.Tensor]) -> None:
    """The same FFN calls alone: each output is left in the runtime's buffer, where the next call overwrites it (a
    model consumes it there, in its residual sum, before the next layer's call)."""
    for i, x in enumerate(xs):
        runtime.forward(i, x)


def measure(runtime: PreparedRuntime, compacts: list[synth.CompactLayer], batch: int, steps: int) -> dict:
    device, layers = runtime.device, len(compacts)
    xs = [torch.from_numpy(synth.make_input(WORKLOAD, batch)).to(device) * (1 + 0.01 * i) for i in range(layers)]
    eager = [torch.empty(batch, WORKLOAD.d_model, device=device) for _ in range(layers)]
    replayed = [torch.empty_like(t) for t in eager]
    for _ in range(3):
        step(runtime, xs, eager)
    torch.cuda.synchronize()

    def timed(run) -> float:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            run()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e3 / steps

    eager_us = timed(lambda: step(runtime, xs, eager))
    calls_us = timed(lambda: calls(runtime, xs))
    bare = torch.cuda.CUDAGraph()
    with torch.cuda.graph(bare):
        calls(runtime, xs)
    calls_graph_us = timed(bare.replay)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(runtime, xs, replayed)
    bitwise = True
    for _ in range(3):  # replays checked against the eager step, with eager work in between
        for t in replayed:
            t.zero_()
        graph.replay()
        step(runtime, xs, eager)
        torch.cuda.synchronize()
        bitwise &= all(torch.equal(a, b) for a, b in zip(eager, replayed))
    graph_us = timed(graph.replay)
    step_bytes = sum(compact_bytes(layer) for layer in compacts)
    return {"batch": batch, "layers": layers, "modes": list(runtime.modes(batch)),
            "calls_us_per_step": round(calls_us, 1), "calls_graph_us_per_step": round(calls_graph_us, 1),
            "calls_us_per_layer": round(calls_us / layers, 2), "ffn_bytes_per_step": step_bytes,
            "hbm_fraction": round(step_bytes / (min(calls_us, calls_graph_us) * 1e-6) / HBM_PEAK, 4),
            "with_copies_eager_us_per_step": round(eager_us, 1), "with_copies_graph_us_per_step": round(graph_us, 1),
            "graph_replays_bitwise": bitwise}


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--batch", default="1,8,16")
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--layers", type=int, default=24)
    parser.add_argument("--tiled", action="store_true", help="the runtime with tiled copies of the stores")
    args = parser.parse_args(argv)
    device = torch.device("cuda", 0)
    compacts = [synth.make_workload_layer(WORKLOAD, seed=WORKLOAD.seed * 1000 + i) for i in range(args.layers)]
    runtime = PreparedRuntime([hip_layer(c, device) for c in compacts], device, tiled=args.tiled)
    for batch in (int(b) for b in args.batch.split(",")):
        print(json.dumps(measure(runtime, compacts, batch, args.steps)), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
