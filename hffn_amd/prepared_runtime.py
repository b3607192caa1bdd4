"""``PreparedRuntime``: the decode launch path, as ``hffn_pythia_cuda.prepared_runtime``
(``runtime/gpu/nvidia/llm/inference/hffn_pythia_cuda/prepared_runtime.py:34-82``).

A decode-sized call of layer ``index`` on N tokens (the gather kernels ``edges`` and ``rows``, the decode GEMVs
``gemv`` or the compact-store MFMA path ``tiles``) launches from a *plan* that the library builds once per (index, N): every argument of the forward but ``x``
and the stream is checked and stored on the library side (``hffn_plan_forward``, ``hffn_plan_gemv``), so a call is
one ctypes call with three arguments (``hffn_plan_launch``) instead of the full argument list and its checks. The
kernels, modes, work buffers, results and the ``calls`` counter are those of ``HFFNRuntime``; MFMA-path calls (large
N) run the control's ``forward``.

Baked device pointers: the eight arrays of the layer (never reassigned, kept alive by the runtime), its planes
(rebuilt in place after a training update, before the next planned launch as before any other) and the work buffers; ``_reserve`` (which reallocates the buffers) and ``force`` release every plan, as the reference drops its
descriptors. ``x`` is never baked. Unlike the reference's descriptors (default stream only), a plan launches on the
device's current stream of each call.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .runtime import MAX_TOKENS, TILES_MAX_TOKENS, HFFNRuntime, _aligned, leading_dim

_GATHER = ("edges", "rows")


class PreparedRuntime(HFFNRuntime):
    """``HFFNRuntime`` whose gather-mode calls launch from per-(layer, N) plans of the HIP library."""

    def __init__(self, layers, device="cuda", dense: bool | None = None, tiled: bool = False) -> None:
        self._plans: dict = {}
        super().__init__(layers, device, dense, tiled)
        self._stream_of = getattr(torch._C, "_cuda_getCurrentRawStream", None)

    def _release_plans(self) -> None:
        plans, self._plans = getattr(self, "_plans", {}), {}
        for entry in plans.values():
            if entry:
                _lib.check(self._lib.hffn_plan_release(entry[0]), "plan release")

    def _reserve(self, n: int) -> None:
        self._release_plans()  # the work buffers move: every plan holding them is stale
        super()._reserve(n)

    def force(self, up, down) -> None:
        super().force(up, down)
        self._release_plans()

    def __del__(self) -> None:
        try:
            self._release_plans()
        except Exception:  # interpreter shutdown: the library may be gone already
            pass

    def _plan(self, index: int, n: int):
        """(handle, up, down) for a gather-mode or decode-GEMV call, or False for a call that takes the control's path."""
        up, down = self.modes(n)
        value_type, *model = self._args[index]
        x_t, act, y_t, y = self._work
        handle = ctypes.c_uint64(0)
        if up == "gemv":
            planes, tensors = self._planes[index], self._tensors[index]
            _lib.check(self._lib.hffn_plan_gemv(value_type, planes["up"].data_ptr(), planes["up_binades"].data_ptr(),
                                                tensors["b_up"].data_ptr(), planes["down"].data_ptr(),
                                                planes["down_binades"].data_ptr(), tensors["b_down"].data_ptr(), act,
                                                self._gemv_work.data_ptr(), 4 * self._gemv_work.numel(), y, self.d_model,
                                                self.d_ff, n, ctypes.byref(handle)),
                       "plan (gemv, gemv)")
            return handle.value, up, down
        if up == "tiles" and n > TILES_MAX_TOKENS:
            return False  # pieces of TILES_MAX_TOKENS tokens: the control's loop
        if up == "tiles":
            entry = self._lib.hffn_plan_tiles if self.tiled else self._lib.hffn_plan_tiles_compact
            _lib.check(entry(value_type, *self._tiles_args(index), self.d_model, self.d_ff, *self._nnz[index], n, ctypes.byref(handle)),
                       "plan (tiles, tiles)")
            return handle.value, up, down
        if up not in _GATHER or down not in _GATHER:
            return False
        _lib.check(self._lib.hffn_plan_forward(_lib.UP_MODES[up], _lib.DOWN_MODES[down], value_type, *model, x_t, act, y_t, y,
                                               self.d_model, self.d_ff, *self._nnz[index], n, leading_dim(n),
                                               ctypes.byref(handle)),
                   f"plan ({up}, {down})")
        return handle.value, up, down

    def forward(self, index: int, x: torch.Tensor) -> torch.Tensor:
        if x.dim() != 2 or x.shape[1] != self.d_model or x.dtype != torch.float32 or x.device != self._y.device or not x.is_contiguous():
            raise ValueError("expected a contiguous float32 [N, d_model] tensor on the runtime's device")
        n = x.shape[0]
        if not 1 <= n <= MAX_TOKENS:
            raise ValueError("unsupported token count")
        if n > self._tokens:
            self._reserve(n)
        key = (index, n)
        entry = self._plans.get(key)
        if entry is None:
            entry = self._plans[key] = self._plan(index, n)
        if entry is False:
            return super().forward(index, x)
        handle, up, down = entry
        if up in ("gemv", "tiles"):
            x = _aligned(x)  # read 16 bytes at a time
            if up == "gemv" and index in self._stale:  # a training update changed the values: rebuild the planes first
                self._densify(self._tensors[index], self._planes[index])
                self._stale.discard(index)
            if up == "tiles":  # likewise the tiled stores
                self._fresh_tiles(index)
        stream = self._stream_of(self.device.index) if self._stream_of else torch.cuda.current_stream(self.device).cuda_stream
        _lib.check(self._lib.hffn_plan_launch(handle, x.data_ptr(), stream), f"forward ({up}, {down})")
        self.calls[up, down] += 1
        return self._y[:n]
