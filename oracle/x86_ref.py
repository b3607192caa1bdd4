"""ctypes binding of the reference x86 AVX2 HFFN kernel (test infrastructure and the CPU baseline of ``bench.py``).

The library ``oracle/_ref/libhffn_x86_ref.so`` is compiled by ``oracle/Makefile`` from
``runtime/cpu/x86/common/kernels/hffn_compact_g4_inference.cpp`` of the reference, with the reference's flags. This
module is this repository's own binder for its C entries (``hffn_compact_g4_inference.cpp:658-701``), following the
calling convention of the reference loader ``runtime/cpu/x86/ffn/inference/hffn/compact.py``:

* routes: ``decode`` for N = 1, ``dual`` for N >= 2 (``compact.py:59-60``);
* batches above 96 tokens run as balanced chunks, multiples of 8 (``compact.py:63-69``);
* hidden groups: T equal parts of ``d_ff`` (``compact.py:85-87``); output groups: balanced by edge count
  (``compact.py:72-82``); the reverse (output-major) schedule comes from ``oracle.transpose``;
* work buffers start on 64-byte boundaries (``compact.py:45-52``); ``y_t`` shares ``x_t`` and ``z`` shares the
  activation buffer, as the reference loader passes them (``compact.py:183-185``).

The kernel is float32-only: a bf16 layer runs with its (exactly representable) float32 values.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

from .transpose import output_major

LIBRARY = Path(__file__).resolve().parent / "_ref" / "libhffn_x86_ref.so"
MAX_BATCH = 96
ALIGNMENT = 64

_P, _I = ctypes.c_void_p, ctypes.c_int


def available() -> bool:
    return LIBRARY.exists()


def aligned_empty(size: int, alignment: int = ALIGNMENT) -> np.ndarray:
    raw = np.empty(size * 4 + alignment, np.uint8)
    start = -raw.ctypes.data % alignment
    return raw[start:start + size * 4].view(np.float32)


def batch_chunks(n: int, max_batch: int | None = MAX_BATCH) -> list[tuple[int, int]]:
    """(start, size) of the consecutive token chunks of a batch of n: balanced, sizes multiples of 8."""
    if not max_batch or n <= max_batch:
        return [(0, n)]
    count = -(-n // max_batch)
    size = -(-(-(-n // count)) // 8) * 8
    return [(start, min(size, n - start)) for start in range(0, n, size)]


def balanced_groups(cost: np.ndarray, threads: int) -> np.ndarray:
    """threads + 1 boundaries over the features; a boundary is placed once the running cost reaches its share."""
    total, boundaries, running, target = int(cost.sum()), [0], 0, 1
    for feature, value in enumerate(cost.tolist()):
        running += int(value)
        while target < threads and running >= round(total * target / threads):
            boundaries.append(feature + 1)
            target += 1
    while len(boundaries) < threads:
        boundaries.append(boundaries[-1])
    boundaries.append(cost.size)
    return np.array(boundaries, dtype=np.int32)


def equal_groups(size: int, threads: int) -> np.ndarray:
    return np.array([(g * size) // threads for g in range(threads + 1)], dtype=np.int32)


class ReferenceKernel:
    """The reference x86 kernel on one compact layer (float32), T threads."""

    def __init__(self, layer, threads: int | None = None, max_batch: int | None = MAX_BATCH):
        if not available():
            raise RuntimeError(f"{LIBRARY} is not built (make -C oracle)")
        self._lib = ctypes.CDLL(str(LIBRARY))
        self._decode = self._lib.hffn_compact_forward_decode_nt_f32
        self._decode.argtypes = [_I] + [_P] * 11 + [_I, _I] + [_P] * 3
        self._dual = self._lib.hffn_compact_forward_dual_nt_f32
        self._dual.argtypes = [_I] + [_P] * 11 + [_I, _I, _I] + [_P] * 6
        self._decode.restype = self._dual.restype = None
        self.threads = threads or max(1, min(len(os.sched_getaffinity(0)), 8))
        self.max_batch = max_batch
        self.d_model, self.d_ff = layer.d_model, layer.d_ff
        f32 = lambda a: np.ascontiguousarray(a, dtype=np.float32)  # noqa: E731
        self._up = (equal_groups(layer.d_ff, self.threads), f32(layer.b_up), np.ascontiguousarray(layer.up_offsets, np.int32),
                    np.ascontiguousarray(layer.up_idx, np.int16), f32(layer.up_val))
        offsets, hidden, weights = output_major(layer.d_model, layer.d_ff, layer.down_offsets, layer.down_idx, f32(layer.down_val))
        self._reverse = (f32(layer.b_down), offsets, hidden, weights, balanced_groups(np.diff(offsets), self.threads))
        self._work: dict[str, np.ndarray] = {}
        self.timing = np.zeros(4, np.int64)

    def _buffer(self, role: str, size: int) -> np.ndarray:
        if role not in self._work or self._work[role].size < size:
            self._work[role] = aligned_empty(size)
        return self._work[role]

    def forward(self, x_nt: np.ndarray) -> np.ndarray:
        """y[N, d_model] for x[N, d_model] (float32, C-contiguous); ``self.timing`` sums the in-kernel phase times."""
        x_nt = np.ascontiguousarray(x_nt, dtype=np.float32)
        n = x_nt.shape[0]
        y = np.empty_like(x_nt)
        a = lambda array: array.ctypes.data  # noqa: E731
        up = [a(v) for v in self._up]
        reverse = [a(v) for v in self._reverse]
        self.timing[:] = 0
        timing = np.zeros(4, np.int64)
        if n == 1:
            act = self._buffer("act", self.d_ff)
            self._decode(self.threads, a(x_nt), *up, *reverse, self.d_model, self.d_ff, a(y), a(act), a(timing))
            self.timing += timing
            return y
        for start, size in batch_chunks(n, self.max_batch):
            x_t = self._buffer("x_t", self.d_model * size)
            act = self._buffer("act", self.d_ff * size)
            self._dual(self.threads, a(x_nt) + start * x_nt.strides[0], *up, *reverse, size, self.d_model, self.d_ff,
                       a(x_t), a(y) + start * y.strides[0], a(x_t), a(act), a(act), a(timing))
            self.timing += timing
        return y
