"""Parity of the HIP runtime on one FFN against a float64 expectation, as ``hffn_cuda.parity``
(``runtime/gpu/nvidia/common/kernels/hffn_cuda/parity.py:16-43``).

For one input, the runtime runs with its policy and with each forced (up, down) kernel pair. Criteria: two
consecutive calls on the same input give the same bits; ``max |y - y64|`` and ``max |y - y64| / max(1, |y64|)`` are
reported for the caller to compare with its tolerance. The pairs are the policy, the four gather pairs (edges or
rows up, edges or rows down) and, when the runtime holds densified planes, the MFMA path and (up to 64 tokens) the
decode GEMVs, and (up to 64 tokens) the compact-store MFMA path.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .runtime import GEMV_MAX_TOKENS, HFFNRuntime

GATHER = ("edges", "rows")
PAIRS = [(None, None)] + [(up, down) for up in GATHER for down in GATHER] + [("mfma", "mfma"), ("gemv", "gemv"), ("tiles", "tiles")]


@dataclass
class Parity:
    """Worst figures over the pairs run: ``error`` the largest absolute distance to the float64 expectation,
    ``relative`` the largest distance scaled by max(1, |expected|), ``repeatable`` whether every pair reproduced its
    own bits on a second call, ``pairs`` the absolute distance of each (up, down) pair."""
    error: float
    relative: float
    repeatable: bool
    pairs: dict


def check(runtime: HFFNRuntime, index: int, x: torch.Tensor, expected: torch.Tensor, pairs=PAIRS) -> Parity:
    """``x`` float32 [N, d_model] on the runtime's device, ``expected`` its float64 oracle output (same device)."""
    scale = expected.abs().clamp(min=1.0)
    result = Parity(0.0, 0.0, True, {})
    try:
        for up, down in pairs:
            if up in ("mfma", "gemv") and not runtime.mfma_available:
                continue
            if up == "tiles" and not runtime.tiles_available:
                continue
            if up in ("gemv", "tiles") and x.shape[0] > GEMV_MAX_TOKENS:
                continue
            runtime.force(up, down)
            y = runtime.forward(index, x).clone()
            result.repeatable &= bool(torch.equal(y, runtime.forward(index, x)))
            distance = (y.double() - expected).abs()
            error = float(distance.max())
            result.pairs[up, down] = error
            result.error = max(result.error, error)
            result.relative = max(result.relative, float((distance / scale).max()))
    finally:
        runtime.force(None, None)
    return result
