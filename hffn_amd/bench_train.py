"""Timing of one HFFN training step (forward with z, backward, compact AdamW) against the dense masked float32 control,
as the reference's FFN training results (``runtime/gpu/nvidia/ffn/training/RESULTS.md``: cells ``<d>_<h>_d<density>``,
N = 1, 8, 64, 512; the control is PyTorch's iso-support step: dense weights, masked gradients, fused AdamW,
``train_step.py:95-121``).

    python -m hffn_amd.bench_train [--cells 512_2048_d020,1024_4096_d050] [--tokens 1,8,64,512] [--steps 50] [--train gather|mfma]

One JSON line per (cell, N): milliseconds per step of each arm (HIP events around ``steps`` steps after warm-up, inputs
resident), their ratio, and the memory each arm keeps for its parameters and optimiser state. Layers are synthetic:
uniform supports of the cell's density, weights ~N(0, 0.02), x ~N(0, 1), gy ~N(0, 0.1).
"""
from __future__ import annotations

import argparse
import json

import numpy as np
import torch
import torch.nn.functional as F

from . import synth
from .ffn import hip_layer
from .runtime import HFFNRuntime
from .train_runtime import HFFNTrainRuntime

HYPER = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2)
CELLS = ("512_2048_d005", "512_2048_d020", "512_2048_d050", "256_1024_d010", "1024_4096_d010", "1024_4096_d050")


def make_cell(name: str, seed: int = 104) -> synth.CompactLayer:
    d, h, density = name.split("_")
    d, h, percent = int(d), int(h), int(density[1:])
    degree = max(1, round(d * percent / 100))
    rng = np.random.default_rng(seed)
    offsets = np.arange(h + 1, dtype=np.int32) * degree
    up_idx = np.concatenate([np.sort(rng.choice(d, degree, replace=False)) for _ in range(h)]).astype(np.int16)
    down_idx = np.concatenate([np.sort(rng.choice(d, degree, replace=False)) for _ in range(h)]).astype(np.int16)
    values = lambda size: (rng.standard_normal(size) * 0.02).astype(np.float32)  # noqa: E731
    return synth.CompactLayer(d, h, synth._groups(h), offsets, up_idx, values(h * degree), np.zeros(h, np.float32), offsets,
                              down_idx, values(h * degree), np.zeros(d, np.float32))


class DenseControl:
    """Dense float32 weights with the support as masks, autograd, masked gradients, fused AdamW."""

    def __init__(self, layer, device) -> None:
        up_owner = np.repeat(np.arange(layer.d_ff), np.diff(layer.up_offsets))
        down_owner = np.repeat(np.arange(layer.d_ff), np.diff(layer.down_offsets))
        w_up = torch.zeros(layer.d_ff, layer.d_model)
        w_up[up_owner, layer.up_idx.astype(np.int64)] = torch.from_numpy(layer.up_val)
        w_down = torch.zeros(layer.d_model, layer.d_ff)
        w_down[layer.down_idx.astype(np.int64), down_owner] = torch.from_numpy(layer.down_val)
        self.masks = ((w_up != 0).float().to(device), None, (w_down != 0).float().to(device), None)
        self.params = [p.to(device).requires_grad_() for p in (w_up, torch.from_numpy(layer.b_up.copy()), w_down,
                                                               torch.from_numpy(layer.b_down.copy()))]
        self.optimiser = torch.optim.AdamW(self.params, fused=True, **HYPER)

    def step(self, x: torch.Tensor, gy: torch.Tensor) -> None:
        w_up, b_up, w_down, b_down = self.params
        xg = x.detach().requires_grad_()
        y = F.linear(F.gelu(F.linear(xg, w_up, b_up), approximate="none"), w_down, b_down)
        y.backward(gy)
        for p, mask in zip(self.params, self.masks):
            if mask is not None:
                p.grad.mul_(mask)
        self.optimiser.step()
        self.optimiser.zero_grad(set_to_none=False)

    def state_bytes(self) -> int:
        state = sum(t.numel() * t.element_size() for s in self.optimiser.state.values() for t in s.values()
                    if torch.is_tensor(t) and t.dim() > 0)
        return state + sum(2 * p.numel() * p.element_size() for p in self.params)


def time_steps(step, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--cells", default=",".join(CELLS))
    parser.add_argument("--tokens", default="1,8,64,512")
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--train", choices=("gather", "mfma"), help="force the forward with z, gz and gx (default: the policy)")
    args = parser.parse_args(argv)
    device = torch.device("cuda", 0)
    tokens = [int(v) for v in args.tokens.split(",")]
    for name in args.cells.split(","):
        layer = make_cell(name)
        train = HFFNTrainRuntime(HFFNRuntime([hip_layer(layer)], device), **HYPER, max_tokens=max(tokens))
        train.forced_train = args.train
        dense = DenseControl(layer, device)
        for n in tokens:
            rng = np.random.default_rng(n)
            x = torch.from_numpy(rng.standard_normal((n, layer.d_model)).astype(np.float32)).to(device)
            gy = torch.from_numpy((0.1 * rng.standard_normal((n, layer.d_model))).astype(np.float32)).to(device)
            train.reserve(n)
            growths = train.growths
            hffn_ms = time_steps(lambda: train.step(0, x, gy), args.steps, args.warmup)
            dense_ms = time_steps(lambda: dense.step(x, gy), args.steps, args.warmup)
            sizes = train.nbytes(0)
            print(json.dumps({"cell": name, "n": n, "hffn_ms": round(hffn_ms, 4), "dense_ms": round(dense_ms, 4),
                              "hffn_over_dense": round(hffn_ms / dense_ms, 3), "train_mode": train.train_mode(n),
                              "grad_mode": train.grad_mode(n), "modes": list(train.modes(n)),
                              "hffn_state_mb": round((sizes["values"] + sizes["gradients"] + sizes["moments"] + sizes["indices"]) / 1e6, 2),
                              "dense_state_mb": round(dense.state_bytes() / 1e6, 2), "growths_in_window": train.growths - growths}),
                  flush=True)
        del train, dense
        torch.cuda.empty_cache()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
