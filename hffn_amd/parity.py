"""Parity of the HIP runtime on one FFN against a float64 expectation, as ``hffn_cuda.parity``
(``runtime/gpu/nvidia/common/kernels/hffn_cuda/parity.py:16-43``).

For one input, the runtime runs with its policy and with each forced (up, down) kernel pair. Criteria: two
consecutive calls on the same input give the same bits; ``max |y - y64|`` and ``max |y - y64| / max(1, |y64|)`` are
reported for the caller to compare with its tolerance. The pairs are the policy, the four gather pairs (edges or
rows up, edges or rows down) and, when the runtime holds densified planes, the MFMA path and (up to 64 tokens) the
decode GEMVs, and (up to 64 tokens) the compact-store MFMA path.

Reported without threshold, as the reference does: ``sequential_bits``, whether the sequential pairs give the same
bits. A pair is sequential when both of its kernels form every output as one running fp32 sum over the slots in
stored order (the reference's up lane/tile with down tiled/blocked). Here the ``rows`` kernels do (a lane holds a
token and walks the row's slots in order; the down side walks the output-major slots in ascending hidden order);
``edges`` sums by wave butterflies, ``tiles``/``mfma``/``gemv`` by MFMA products. With ``SEQUENTIAL`` = the one pair
(rows, rows), the field also asks that the pair's bits do not depend on how the call batches tokens: the pair's
output for the whole input equals, token for token, its outputs for the input's two halves run as separate calls.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .runtime import GEMV_MAX_TOKENS, HFFNRuntime

GATHER = ("edges", "rows")
PAIRS = [(None, None)] + [(up, down) for up in GATHER for down in GATHER] + [("mfma", "mfma"), ("gemv", "gemv"), ("tiles", "tiles")]
SEQUENTIAL = (("rows", "rows"),)  # pairs whose kernels sum each output in stored slot order


@dataclass
class Parity:
    """Worst figures over the pairs run: ``error`` the largest absolute distance to the float64 expectation,
    ``relative`` the largest distance scaled by max(1, |expected|), ``repeatable`` whether every pair reproduced its
    own bits on a second call, ``sequential_bits`` whether the sequential pairs run gave the same bits (and the same
    bits when the input was split in two calls; True when none ran), ``pairs`` the absolute distance of each
    (up, down) pair."""
    error: float
    relative: float
    repeatable: bool
    sequential_bits: bool = True
    pairs: dict = field(default_factory=dict)


def check(runtime: HFFNRuntime, index: int, x: torch.Tensor, expected: torch.Tensor, pairs=PAIRS) -> Parity:
    """``x`` float32 [N, d_model] on the runtime's device, ``expected`` its float64 oracle output (same device)."""
    scale = expected.abs().clamp(min=1.0)
    result, sequential = Parity(0.0, 0.0, True), None
    try:
        for up, down in pairs:
            if up in ("mfma", "gemv") and not runtime.mfma_available:
                continue
            if up == "tiles" and not runtime.tiles_available:
                continue
            if up == "gemv" and x.shape[0] > GEMV_MAX_TOKENS:
                continue
            runtime.force(up, down)
            y = runtime.forward(index, x).clone()
            result.repeatable &= bool(torch.equal(y, runtime.forward(index, x)))
            if (up, down) in SEQUENTIAL:
                if sequential is None:
                    sequential = y
                result.sequential_bits &= bool(torch.equal(y, sequential))
                half = x.shape[0] // 2
                if half:
                    first = runtime.forward(index, x[:half].contiguous()).clone()
                    second = runtime.forward(index, x[half:].contiguous())
                    result.sequential_bits &= bool(torch.equal(first, y[:half]) and torch.equal(second, y[half:]))
            distance = (y.double() - expected).abs()
            error = float(distance.max())
            result.pairs[up, down] = error
            result.error = max(result.error, error)
            result.relative = max(result.relative, float((distance / scale).max()))
    finally:
        runtime.force(None, None)
    return result
