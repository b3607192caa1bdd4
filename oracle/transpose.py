"""Output-major transpose of a hidden-major down store (test infrastructure; see ``oracle/__init__.py``).

For output o, the slots s with ``down_idx[s] == o`` in increasing s; ``out_hidden`` holds the owner neuron of each such
slot and ``out_val`` its value (``runtime/gpu/nvidia/common/kernels/hffn_cuda/runtime.py:55-67``, and the same
transpose in ``runtime/cpu/x86/ffn/inference/hffn/compact.py:90-104``).
"""
from __future__ import annotations

import numpy as np


def output_major(d_model: int, d_ff: int, down_offsets: np.ndarray, down_idx: np.ndarray, down_val: np.ndarray):
    """numpy: stable argsort of the output index, bincount prefix for the offsets."""
    index = down_idx.astype(np.int64)
    order = np.argsort(index, kind="stable")
    out_offsets = np.zeros(d_model + 1, dtype=np.int32)
    out_offsets[1:] = np.cumsum(np.bincount(index, minlength=d_model))
    owner = np.repeat(np.arange(d_ff), np.diff(down_offsets.astype(np.int64)))
    return out_offsets, owner[order].astype(np.int16), np.ascontiguousarray(down_val[order])


def output_major_loops(d_model: int, d_ff: int, down_offsets, down_idx, down_val):
    """Pure Python: append every slot, in hidden-major order, to the bucket of its output."""
    buckets = [[] for _ in range(d_model)]
    offsets = [int(v) for v in down_offsets]
    for r in range(d_ff):
        for s in range(offsets[r], offsets[r + 1]):
            buckets[int(down_idx[s])].append((r, s))
    out_offsets = np.zeros(d_model + 1, dtype=np.int32)
    hidden, slots = [], []
    for o, bucket in enumerate(buckets):
        out_offsets[o + 1] = out_offsets[o] + len(bucket)
        hidden.extend(r for r, _ in bucket)
        slots.extend(s for _, s in bucket)
    values = np.asarray(down_val)[np.asarray(slots, dtype=np.int64)] if slots else np.asarray(down_val)[:0]
    return out_offsets, np.asarray(hidden, dtype=np.int16), values
