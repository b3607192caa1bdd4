"""HFFN forward runtime on MI355X: a stack of FFNs of one shape (the FFNs of one model, or one isolated FFN).

Drop-in for ``hffn_cuda.runtime`` (``runtime/gpu/nvidia/common/kernels/hffn_cuda/runtime.py``): same classes, fields,
methods, counters and errors. One call runs the whole block of N tokens of one FFN through the HIP library
(``libhffn_amd.so``, C ABI in ``include/hffn_amd.h``): an up kernel (one wave per hidden neuron, bias and exact GELU
fused) then a down kernel (one wave per output feature, over the output-major store), with the layout transposes
the chosen shapes need.

Kernel shapes (the build's own policy, ``up_mode``/``down_mode``):

* ``edges`` - lanes over a row's slots, tokens in registers, input staged in LDS; decode-sized N (N <= 32).
* ``tiles`` - the compact-store MFMA path (up and down together, 1-64 tokens): each side read once, from the compact
  rows through a table of row bounds (default) or from a tiled copy (``tiled=True``: the compact slots regrouped at
  load by 16-row tile and 512-wide sub-chunk of K, interleaved 16-bit fields), densified per block in LDS and
  multiplied on 16x16x32 MFMAs.
* ``rows``  - lanes over tokens (1, 2 or 4 per lane), slots walked in order; large N on layers without the MFMA path.
* ``mfma``  - tile-densified split-fp16 MFMA GEMMs over dense planes (up and down together) on high-density layers
  (density at least ``MFMA_MIN_DENSITY``, ``d_model`` and ``d_ff`` multiples of 256), above 64 tokens.
* ``gemv``  - decode GEMVs over the same planes (1-64 tokens); never chosen by the policy (the planes are kept for
  large token counts), run when forced.

The policy reads the compact store up to 64 tokens: ``edges`` (up to 32 tokens) or ``tiles``, whichever has the least
estimated time (``decode_mode``); above 64 tokens the MFMA path where the layer has planes, else ``tiles`` in pieces of
64 tokens or ``rows``, whichever has the least estimated time (``pieces_us``, ``rows_us``: the tiles path reads the
store once per piece, the lane-per-token kernels read an input row per slot and token, so the tiles path takes the
larger layers, e.g. the 1.4B layer at 20 %, 59 against 213 us at 65 tokens and 1.32 against 2.00 ms at 2048, and the
lane-per-token kernels the smallest, e.g. the 70M layer at 20 % from 65 tokens on, 38.9 against 44.0 us). The dense
planes (4 bytes per weight for float32 values, 2 for bfloat16) are built only for layers of at least
``MFMA_MIN_DENSITY`` unless asked for (``dense=True``). Per call on the Pythia-410M layer at 50 % (12 rotating
copies, MI355X, HFFNRuntime.forward, forced pairs, compact rows): N = 1: edges 12.9 us, tiles 17.8; N = 4: edges
14.3, tiles 17.5; N = 16: tiles 17.8, edges 39.0; N = 32: tiles 21.5; N = 2048: mfma 110-116 us. On the 1.4B layer
(bfloat16, 20 %): edges 13.0, 14.4, 17.9 us at N = 1, 2, 4 (tiles 19.0, 19.0, 19.3), tiles 23.0 and 31.5 us at 16
and 32 (edges 59.5 at 16).

Model arrays stay on the device. Work buffers are dense, shared by all layers, sized for the largest N seen and
reused. Kernels are queued on PyTorch's current stream of the device, so they run in call order with the PyTorch
operations around them (the reference requires the default stream; any current stream is accepted here).
"""
from __future__ import annotations

import ctypes
import math
from collections import Counter
from dataclasses import dataclass

import torch

from . import _lib

UP_MODES = ("edges", "rows", "mfma", "gemv", "tiles")
DOWN_MODES = ("edges", "rows", "mfma", "gemv", "tiles")
PAIR_MODES = ("mfma", "gemv", "tiles")  # up and down run together (token-major activations of their own)
PLANES_MODES = ("mfma", "gemv")         # the paths over densified planes
GEMV_MAX_TOKENS = 64      # the planes GEMVs' largest call
TILES_MAX_TOKENS = 64     # the compact-store MFMA path's largest call
EDGES_MAX_TOKENS = 32     # the policy's last N for the lane-per-slot shapes
EDGES_PASS_TOKENS = 8     # tokens one pass of the lane-per-slot kernels takes
MFMA_MIN_DENSITY = 0.5    # the lowest support density whose layers get dense planes by default (the MFMA path)
# The policy's time estimates (µs per call), fitted to forced-pair timings of HFFNRuntime.forward on MI355X (layer
# copies rotated so that every call reads HBM; the 70M/20 %, 410M/10 % and 50 %, 1.4B/20 % bf16 and 2.8B/80 % bf16
# layers at 1-32 tokens: the faster path at every one of the 50 points). Lane-per-slot kernels, per pass of up to 8
# tokens (a pass's width: 1, 2, 4 or 8): the larger of a floor of round trips and launches (EDGES_FLOOR_US of the
# width, plus EDGES_SLOT_TOKEN_US per stored slot of both sides and token of the width) and the stores' stream
# (EDGES_BYTE_US per stored byte, ~3.2 TB/s); a pass whose activations exceed the down kernel's LDS stage
# (EDGES_STAGE_BYTES) gathers them from L2, EDGES_GATHER times slower. Compact-store MFMA path: the larger of a floor
# that grows with the width of the layer (TILES_FLOOR_US + TILES_WIDTH_US per doubling of d_ff from 1024; below
# 2048, the narrowest fitted, that layer's floor) and the stores' stream (TILES_BYTE_US per byte, ~2.5 TB/s), plus up
# to (TILES_FILL_US + TILES_FILL_SLOT_US per slot) as the first 16-token tile fills, plus (TILES_TILE_US +
# TILES_TILE_SLOT_US per slot) per further 16-token tile.
EDGES_FLOOR_US = {1: 11.8, 2: 11.8, 4: 11.8, 8: 13.2}
EDGES_SLOT_TOKEN_US, EDGES_BYTE_US = 0.2e-6, 0.315e-6
EDGES_STAGE_BYTES, EDGES_GATHER = 131072, 2.3
TILES_FLOOR_US, TILES_WIDTH_US, TILES_BYTE_US = 11.9, 2.47, 0.406e-6
TILES_FILL_US, TILES_FILL_SLOT_US = 2.0, 0.07e-6
TILES_TILE_US, TILES_TILE_SLOT_US = 4.5, 0.17e-6
TILES_TIE = 1.05  # the tiles path wins estimates within 5 % of the lane-per-slot kernels' (its cost is flat in N)
# Lane-per-token kernels above 64 tokens: ROWS_CALL_US per call plus ROWS_SLOT_US per stored slot (both sides) and token
# (each slot reads its input row of every token from L2), fitted to forced-pair timings of the 70M/20 %, 410M/50 % and
# 1.4B/20 % bf16 layers at 65-2048 tokens; against it the tiles path in pieces of 64 tokens (one tiles_us each).
ROWS_CALL_US, ROWS_SLOT_US = 30.0, 0.148e-6
MAX_TOKENS = 1 << 18      # runtime/gpu/nvidia/common/kernels/hffn_cuda/runtime.py:26
# The reference's policy constants (runtime.py:24-25), with this policy's meaning: COOP_MAX_TOKENS, the largest N the
# policy may run on the cooperative (lane-per-slot, wave-reduced) kernels; BLOCK_MAX_WIDTH, the widest d_ff up to which
# the down choice is the same as for narrower FFNs - every d_ff the 16-bit hidden ids of the output-major store can
# address, since the choice here does not depend on d_ff.
COOP_MAX_TOKENS = EDGES_MAX_TOKENS
BLOCK_MAX_WIDTH = 1 << 15

_VALUE_TYPES = {torch.float32: _lib.VALUE_F32, torch.bfloat16: _lib.VALUE_BF16}


def up_mode(n: int, d_model: int | None = None) -> str:
    """Up kernel shape for N tokens: ``edges`` up to ``EDGES_MAX_TOKENS`` (when its LDS stage fits), else ``rows``."""
    if n <= EDGES_MAX_TOKENS and (d_model is None or edges_supported(d_model, n)):
        return "edges"
    return "rows"


def down_mode(n: int, d_ff: int | None = None) -> str:
    """Down kernel shape for N tokens (``d_ff`` kept for the reference signature, ``runtime.py:33``)."""
    return "edges" if n <= EDGES_MAX_TOKENS else "rows"


def edges_supported(d_model: int, n: int) -> bool:
    return bool(_lib.load().hffn_edges_supported(d_model, n))


@dataclass(frozen=True)
class StoreShape:
    """What the path estimates read of a layer: the stored slots of both sides, their bytes (int16 indices and the
    values) and d_ff (the activations the down kernels read, the width of the tiles path's blocks)."""
    slots: int
    bytes: int
    d_ff: int


def _width(tokens: int) -> int:
    return 1 << (tokens - 1).bit_length()  # 1, 2, 4 or 8 tokens per lane-per-slot pass


def edges_us(n: int, shape: StoreShape) -> float:
    """Estimated µs of a call on the lane-per-slot kernels: passes of up to 8 tokens."""
    total = 0.0
    while n > 0:
        tokens = min(n, EDGES_PASS_TOKENS)
        width = _width(tokens)
        cost = max(EDGES_FLOOR_US[width] + EDGES_SLOT_TOKEN_US * shape.slots * width, EDGES_BYTE_US * shape.bytes)
        if shape.d_ff * width * 4 > EDGES_STAGE_BYTES:
            cost *= EDGES_GATHER
        total += cost
        n -= tokens
    return total


def tiles_us(n: int, shape: StoreShape) -> float:
    """Estimated µs of a call on the compact-store MFMA path (N <= 64)."""
    floor = TILES_FLOOR_US + TILES_WIDTH_US * math.log2(max(shape.d_ff, 2048) / 1024)
    return (max(floor, TILES_BYTE_US * shape.bytes) + (TILES_FILL_US + TILES_FILL_SLOT_US * shape.slots) * min(n - 1, 15) / 15
            + (TILES_TILE_US + TILES_TILE_SLOT_US * shape.slots) * ((n - 1) // 16))


def rows_us(n: int, shape: StoreShape) -> float:
    """Estimated µs of a call on the lane-per-token kernels above 64 tokens."""
    return ROWS_CALL_US + ROWS_SLOT_US * shape.slots * n


def pieces_us(n: int, shape: StoreShape) -> float:
    """Estimated µs of N tokens on the tiles path, in calls of up to ``TILES_MAX_TOKENS`` tokens."""
    whole, rest = divmod(n, TILES_MAX_TOKENS)
    return whole * tiles_us(TILES_MAX_TOKENS, shape) + (tiles_us(rest, shape) if rest else 0.0)


def decode_mode(n: int, shape: StoreShape, edges: bool, tiles: bool) -> str | None:
    """The compact-store path of least estimated time for N <= 64 tokens: ``edges`` (up to ``EDGES_MAX_TOKENS``, when
    ``edges``: its LDS stage fits) or ``tiles`` (when ``tiles``: the layer has tiled stores; it also takes estimates
    within ``TILES_TIE`` of the lane-per-slot kernels'); None when neither applies."""
    options = {}
    if edges and n <= EDGES_MAX_TOKENS:
        options["edges"] = edges_us(n, shape)
    if tiles and n <= TILES_MAX_TOKENS:
        options["tiles"] = tiles_us(n, shape) / TILES_TIE
    return min(options, key=options.get) if options else None


def mfma_streamed(n: int, d_model: int, d_ff: int) -> bool:
    """Whether both MFMA projections of N tokens run on the streamed GEMM (``hffn_mfma_streamed``)."""
    status = _lib.load().hffn_mfma_streamed(n, d_model, d_ff)
    if status < 0:
        _lib.check(status, "mfma_streamed")
    return status == 1


def leading_dim(n: int) -> int:
    """Leading dimension of the feature-major work buffers for N tokens: a multiple of 4, and of 8 above 4 tokens
    (the edges shapes read 8-token vectors)."""
    return (n + 3) // 4 * 4 if n <= 4 else (n + 7) // 8 * 8


def _device(device: str | torch.device | None) -> torch.device:
    device = torch.device("cuda" if device is None else device)
    if device.type != "cuda" or device.index not in (None, 0):
        raise ValueError("the HFFN HIP runtime runs on cuda:0")
    if not torch.cuda.is_available():
        raise RuntimeError("the HFFN HIP runtime needs a ROCm GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda", 0)


def _value_type(tensor: torch.Tensor, name: str) -> int:
    try:
        return _VALUE_TYPES[tensor.dtype]
    except KeyError:
        raise ValueError(f"{name} must be float32 or bfloat16, not {tensor.dtype}") from None


def _aligned(tensor: torch.Tensor, alignment: int = 16) -> torch.Tensor:
    """The tensor itself when its data starts on an `alignment`-byte boundary (the edges kernels load 4 slots at a
    time), else an aligned copy."""
    return tensor if tensor.data_ptr() % alignment == 0 else tensor.clone()


def _rows_strictly_increasing(offsets: torch.Tensor, index: torch.Tensor) -> bool:
    """Whether every row's indices increase strictly (distinct, sorted): what the densified planes assume."""
    if index.numel() < 2:
        return True
    step = index[1:].int() - index[:-1].int()
    starts = offsets[1:-1].long()
    starts = starts[(starts > 0) & (starts < index.numel())] - 1
    step[starts] = 1
    return bool((step > 0).all())


def _check_side(name: str, offsets: torch.Tensor, index: torch.Tensor, values: torch.Tensor, rows: int, width: int) -> None:
    """Offsets int32[rows + 1] from 0 to nnz, non-decreasing; int16 indices in [0, width); one value per index."""
    if offsets.dtype != torch.int32 or offsets.dim() != 1 or offsets.numel() != rows + 1:
        raise ValueError(f"{name}: offsets must be int32[{rows + 1}]")
    if index.dtype != torch.int16 or index.dim() != 1 or values.dim() != 1 or values.numel() != index.numel():
        raise ValueError(f"{name}: expected int16 indices and one value per index")
    if int(offsets[0]) != 0 or int(offsets[-1]) != index.numel() or bool((offsets.diff() < 0).any()):
        raise ValueError(f"{name}: offsets must run from 0 to nnz without decreasing")
    if index.numel() and (int(index.min()) < 0 or int(index.max()) >= width):
        raise ValueError(f"{name}: index out of [0, {width})")


@dataclass(frozen=True)
class HFFNLayer:
    """What the kernels read for one FFN: the up arrays per hidden neuron and the down edges in output order
    (fields of ``runtime/gpu/nvidia/common/kernels/hffn_cuda/runtime.py:41-53``; values float32, or bfloat16 for a
    bf16 store, the same dtype on both sides)."""
    d_model: int
    d_ff: int
    b_up: torch.Tensor         # float32[d_ff]
    up_offsets: torch.Tensor   # int32[d_ff + 1]
    up_idx: torch.Tensor       # int16[nnz_up], input feature of each slot
    up_val: torch.Tensor       # float32|bfloat16[nnz_up]
    b_down: torch.Tensor       # float32[d_model]
    out_offsets: torch.Tensor  # int32[d_model + 1]
    out_hidden: torch.Tensor   # int16[nnz_down], hidden neuron of each edge (ascending within an output)
    out_val: torch.Tensor      # float32|bfloat16[nnz_down]

    @classmethod
    def from_hidden_major(cls, d_model: int, d_ff: int, b_up: torch.Tensor, up_offsets: torch.Tensor, up_idx: torch.Tensor,
                          up_val: torch.Tensor, b_down: torch.Tensor, down_offsets: torch.Tensor, down_idx: torch.Tensor,
                          down_val: torch.Tensor, device: str | torch.device | None = None) -> "HFFNLayer":
        """From the canonical hidden-major storage: for neuron r, its up slots and its down slots (output feature of
        each slot in ``down_idx``) at ``[offsets[r], offsets[r + 1])``. The up arrays are kept as given (moved to the
        device); the output-major down store is built on the device by ``hffn_output_major`` (a stable counting sort
        of the slots by output, bitwise the ``argsort(stable)`` transpose of ``runtime.py:55-67``)."""
        dev = _device(device)
        _check_side("up", up_offsets, up_idx, up_val, d_ff, d_model)
        _check_side("down", down_offsets, down_idx, down_val, d_ff, d_model)
        if up_val.dtype != down_val.dtype:
            raise ValueError("up_val and down_val must have the same dtype")
        value_type = _value_type(down_val, "down_val")
        if b_up.dtype != torch.float32 or b_up.numel() != d_ff or b_down.dtype != torch.float32 or b_down.numel() != d_model:
            raise ValueError("b_up must be float32[d_ff] and b_down float32[d_model]")
        moved = [t.to(dev).contiguous() for t in (b_up, up_offsets, up_idx, up_val, b_down, down_offsets, down_idx, down_val)]
        b_up, up_offsets, up_idx, up_val, b_down, down_offsets, down_idx, down_val = moved
        nnz = down_idx.numel()
        out_offsets = torch.empty(d_model + 1, dtype=torch.int32, device=dev)
        out_hidden = torch.empty(nnz, dtype=torch.int16, device=dev)
        out_val = torch.empty(nnz, dtype=down_val.dtype, device=dev)
        lib = _lib.load()
        needed = _lib.ctypes.c_uint64(0)
        _lib.check(lib.hffn_output_major_workspace(nnz, d_model, _lib.ctypes.byref(needed)), "output-major workspace")
        workspace = torch.empty(max(needed.value, 4), dtype=torch.uint8, device=dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        _lib.check(lib.hffn_output_major(value_type, down_offsets.data_ptr(), down_idx.data_ptr(), down_val.data_ptr(),
                                         d_model, d_ff, nnz, out_offsets.data_ptr(), out_hidden.data_ptr(),
                                         out_val.data_ptr(), workspace.data_ptr(), workspace.numel(), stream),
                   "output-major build")
        torch.cuda.current_stream(dev).synchronize()  # the workspace is released on return
        return cls(d_model, d_ff, b_up, up_offsets, up_idx, up_val, b_down, out_offsets, out_hidden, out_val)

    def model_bytes(self) -> int:
        return sum(value.numel() * value.element_size() for value in vars(self).values() if isinstance(value, torch.Tensor))


_ARRAYS = ("b_up", "up_offsets", "up_idx", "up_val", "b_down", "out_offsets", "out_hidden", "out_val")


class HFFNRuntime:
    """``HFFNRuntime`` of ``runtime/gpu/nvidia/common/kernels/hffn_cuda/runtime.py:76-163`` on the HIP library."""

    def __init__(self, layers: list[HFFNLayer], device: str | torch.device = "cuda", dense: bool | None = None,
                 tiled: bool = False) -> None:
        """``dense``: build the dense planes of the MFMA path and the decode GEMVs (``d_model`` and ``d_ff`` multiples of
        256, distinct sorted indices per row): None (default) for layers of at least ``MFMA_MIN_DENSITY`` only, True
        whenever the shapes qualify (the policy still takes them only at that density), False never. ``tiled``: the
        tiles path reads the compact rows themselves through a small table of row bounds (False, the default: one
        resident copy of each store, the layer's own) or a tiled copy of each layer's store built at construction
        (True: its interleaved groups make the tiles calls 5-9 % faster, for a second copy of the store); both give the
        same bits."""
        self.device = _device(device)
        self.tiled = tiled
        self.layers = layers
        self.d_model, self.d_ff = layers[0].d_model, layers[0].d_ff
        if any((layer.d_model, layer.d_ff) != (self.d_model, self.d_ff) for layer in layers):
            raise ValueError("all layers of a runtime share d_model and d_ff")
        if self.d_model % 16:
            raise ValueError("d_model must be a multiple of 16")
        self._lib = _lib.load()
        self._tensors = []
        self._args = []
        self._nnz = []
        for layer in layers:
            tensors = {name: _aligned(getattr(layer, name).to(self.device).contiguous()) for name in _ARRAYS}
            _check_side("up", tensors["up_offsets"], tensors["up_idx"], tensors["up_val"], self.d_ff, self.d_model)
            _check_side("down", tensors["out_offsets"], tensors["out_hidden"], tensors["out_val"], self.d_model, self.d_ff)
            if tensors["up_val"].dtype != tensors["out_val"].dtype:
                raise ValueError("up_val and out_val must have the same dtype")
            if tensors["b_up"].numel() != self.d_ff or tensors["b_down"].numel() != self.d_model:
                raise ValueError("bias dimensions do not match d_model/d_ff")
            self._tensors.append(tensors)
            self._args.append((_value_type(tensors["up_val"], "up_val"),
                               *(tensors[name].data_ptr() for name in ("up_offsets", "up_idx", "up_val", "b_up",
                                                                       "out_offsets", "out_hidden", "out_val", "b_down"))))
            self._nnz.append((tensors["up_idx"].numel(), tensors["out_hidden"].numel()))
        self._slots = max(layer.up_idx.numel() + layer.out_hidden.numel() for layer in layers)
        self.density = self._slots / (2 * self.d_model * self.d_ff)
        self._store = StoreShape(self._slots, self._slots * (2 + self._tensors[0]["up_val"].element_size()), self.d_ff)
        self._planes: list[dict] | None = None
        self._stale: set[int] = set()   # layers whose values changed since their planes were built
        self._tiles_stale: set[int] = set()  # ... since their tiled stores were built
        self._tiles: list[dict] | None = None
        self._tiles_work = torch.empty(1, device=self.device)
        if self._tiles_eligible():
            self._tiles = [self._tiles_build(tensors) for tensors in self._tensors]
            value_type = self._args[0][0]
            words = max(_lib.query_bytes(self._lib.hffn_tiles_workspace, value_type, TILES_MAX_TOKENS, self.d_model, self.d_ff,
                                         *nnz) for nnz in self._nnz) // 4
            self._tiles_work = torch.empty(words, device=self.device)  # the per-chunk partial sums
        self._gemv_work = torch.empty(1, device=self.device)
        if (dense or (dense is None and self.density >= MFMA_MIN_DENSITY)) and self._mfma_eligible():
            self._planes = [self._densify(tensors) for tensors in self._tensors]
            words = (_lib.query_bytes(self._lib.hffn_gemv_workspace, self.d_model, self.d_ff) + 3) // 4
            self._gemv_work = torch.empty(words, device=self.device)  # the decode GEMVs' k-split partial sums
        self._policy: dict[int, tuple[str, str]] = {}  # N -> the policy's (up, down)
        self.forced_up: str | None = None
        self.forced_down: str | None = None
        self.calls: Counter = Counter()
        self._tokens = 0
        self._reserve(1)

    # ------------------------------------------------------------------- compact-store MFMA path (decode sizes)

    def _rows_sorted(self) -> bool:
        if not hasattr(self, "_sorted"):
            self._sorted = all(_rows_strictly_increasing(t["up_offsets"], t["up_idx"]) and
                               _rows_strictly_increasing(t["out_offsets"], t["out_hidden"]) for t in self._tensors)
        return self._sorted

    def _tiles_eligible(self) -> bool:
        return self.d_model % 16 == 0 and self.d_ff % 8 == 0 and self._rows_sorted()

    def _tiles_build(self, tensors: dict, tiles: dict | None = None) -> dict:
        """The tiled stores of both sides (``hffn_tiles_build``): each side's slots regrouped by 16-row tile and 512-wide
        sub-chunk of K, with their table; or, for ``tiled=False``, each side's table of row bounds over the compact rows
        (``hffn_tiles_table_build``). Rebuilt into ``tiles`` when given (same sizes: allocates nothing)."""
        stream = torch.cuda.current_stream(self.device).cuda_stream
        value_type = _value_type(tensors["up_val"], "up_val")
        tiles = {} if tiles is None else tiles
        for side, rows, k, names in (("up", self.d_ff, self.d_model, ("up_offsets", "up_idx", "up_val")),
                                     ("down", self.d_model, self.d_ff, ("out_offsets", "out_hidden", "out_val"))):
            offsets, index, values = (tensors[name] for name in names)
            if not self.tiled:
                if side not in tiles:
                    entries = ctypes.c_uint64(0)
                    _lib.check(self._lib.hffn_tiles_table_size(value_type, rows, k, ctypes.byref(entries)), f"tiles table size {side}")
                    tiles[side] = torch.empty(entries.value, dtype=torch.int32, device=self.device)
                _lib.check(self._lib.hffn_tiles_table_build(value_type, offsets.data_ptr(), index.data_ptr(), values.data_ptr(), rows, k,
                                                            tiles[side].data_ptr(), stream), f"tiles table {side}")
                continue
            store_bytes, entries = ctypes.c_uint64(0), ctypes.c_uint64(0)
            _lib.check(self._lib.hffn_tiles_store_size(value_type, rows, k, index.numel(), ctypes.byref(store_bytes),
                                                       ctypes.byref(entries)), f"tiles store size {side}")
            if side not in tiles:
                tiles[side] = torch.empty(store_bytes.value, dtype=torch.uint8, device=self.device)
                tiles[f"{side}_table"] = torch.empty(entries.value, dtype=torch.int32, device=self.device)
            store, table = tiles[side], tiles[f"{side}_table"]
            _lib.check(self._lib.hffn_tiles_build(value_type, offsets.data_ptr(), index.data_ptr(), values.data_ptr(), rows, k,
                                                  index.numel(), store.data_ptr(), store.numel(), table.data_ptr(), stream),
                       f"tiles build {side}")
        return tiles

    def tiles_bytes(self) -> int:
        """Bytes held for the tiles path beyond the compact store: the tiled stores and their tables, or (``tiled=False``)
        the tables of row bounds; 0 without it."""
        if self._tiles is None:
            return 0
        return sum(t.numel() * t.element_size() for tiles in self._tiles for t in tiles.values())

    @property
    def tiles_available(self) -> bool:
        return self._tiles is not None

    # -------------------------------------------------------------------------------- tile-densified MFMA path

    def _mfma_eligible(self) -> bool:
        return bool(self._lib.hffn_mfma_supported(self.d_model, self.d_ff)) and self._rows_sorted()

    def _densify(self, tensors: dict, planes: dict | None = None) -> dict:
        """fp16 hi/lo planes (and per-row binades) of W_up [d_ff, d_model] and W_down [d_model, d_ff], built on the
        device from the compact store (into ``planes`` when given: a rebuild allocates nothing)."""
        value_type = _value_type(tensors["up_val"], "up_val")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        fresh = planes is None
        planes = {} if fresh else planes
        for side, rows, k, names in (("up", self.d_ff, self.d_model, ("up_offsets", "up_idx", "up_val")),
                                     ("down", self.d_model, self.d_ff, ("out_offsets", "out_hidden", "out_val"))):
            if fresh:
                size = _lib.query_bytes(self._lib.hffn_dense_planes_bytes, rows, k)
                plane = torch.empty(size // 2, dtype=torch.float16, device=self.device)
                binades = torch.empty(rows, dtype=torch.int32, device=self.device)
            else:
                plane, binades = planes[side], planes[f"{side}_binades"]
            offsets, index, values = (tensors[name] for name in names)
            _lib.check(self._lib.hffn_densify(value_type, offsets.data_ptr(), index.data_ptr(), values.data_ptr(), rows, k,
                                              plane.data_ptr(), binades.data_ptr(), stream), f"densify {side}")
            planes[side] = plane
            planes[f"{side}_binades"] = binades
        return planes

    def invalidate_planes(self, index: int) -> None:
        """The compact values of layer ``index`` changed in place (a training update): its densified planes and its tiled
        stores are rebuilt, in place, before a call next reads them (a training loop rebuilds nothing it does not read)."""
        if self._planes is not None:
            self._stale.add(index)
        if self._tiles is not None:
            self._tiles_stale.add(index)

    def _fresh_tiles(self, index: int) -> None:
        if index in self._tiles_stale:
            self._tiles_build(self._tensors[index], self._tiles[index])
            self._tiles_stale.discard(index)

    @property
    def mfma_available(self) -> bool:
        return self._planes is not None

    def dense_bytes(self) -> int:
        """Bytes of the densified planes held for the MFMA path (0 without it)."""
        if self._planes is None:
            return 0
        return sum(t.numel() * t.element_size() for planes in self._planes for t in planes.values())

    def force(self, up: str | None, down: str | None) -> None:
        """Diagnostic: fix the up and/or the down kernel regardless of N (None: the policy). The planes paths run up and
        down together: ``mfma`` and ``gemv`` are forced as pairs (``gemv`` serves 1-64 tokens)."""
        if up not in (None, *UP_MODES) or down not in (None, *DOWN_MODES):
            raise ValueError("unknown kernel mode")
        if up == "edges" and not edges_supported(self.d_model, 1):
            raise ValueError("the edges up shape cannot stage this d_model")
        for pair in PAIR_MODES:
            if (up == pair) != (down == pair):
                raise ValueError(f"the {pair} path runs up and down together: force ('{pair}', '{pair}')")
        if up in PLANES_MODES and self._planes is None:
            raise ValueError(f"the {up} path is not available for these layers")
        if up == "tiles" and self._tiles is None:
            raise ValueError("the tiles path needs d_model % 16 == 0, d_ff % 8 == 0 and strictly increasing indices per row")
        self.forced_up, self.forced_down = up, down

    def _reserve(self, n: int) -> None:
        self._tokens = n
        ld = leading_dim(n)
        self._x_t = torch.empty(self.d_model * ld, device=self.device)   # [d_model, ld]
        self._act = torch.empty(self.d_ff * ld, device=self.device)      # [d_ff, ld]
        self._y_t = torch.empty(self.d_model * ld, device=self.device)   # [d_model, ld]
        self._y = torch.empty(n, self.d_model, device=self.device)
        words = 1
        if self._planes is not None:
            words = (_lib.query_bytes(self._lib.hffn_mfma_workspace, n, self.d_model, self.d_ff) + 3) // 4
        # zero-filled once: the split-K counters it holds start at zero and every call leaves them at zero
        self._mfma_work = torch.zeros(words, dtype=torch.int32, device=self.device)
        self._work = (self._x_t.data_ptr(), self._act.data_ptr(), self._y_t.data_ptr(), self._y.data_ptr())

    def workspace_bytes(self) -> int:
        return 4 * (self._x_t.numel() + self._act.numel() + self._y_t.numel() + self._y.numel() + self._mfma_work.numel() +
                    self._gemv_work.numel() + self._tiles_work.numel())

    def modes(self, n: int) -> tuple[str, str]:
        """The (up, down) shapes a call of N tokens takes (forced ones first). The policy's choice depends on N and the
        layers only, so it is worked out once per N (the library queries behind it are ctypes calls)."""
        chosen = self._policy.get(n) if self.forced_up is None and self.forced_down is None else None
        if chosen is None:
            chosen = self._modes(n)
            if self.forced_up is None and self.forced_down is None:
                self._policy[n] = chosen
        return chosen

    def _modes(self, n: int) -> tuple[str, str]:
        edges = edges_supported(self.d_model, n)
        if self.forced_up is None and self.forced_down is None:
            if n <= TILES_MAX_TOKENS:
                mode = decode_mode(n, self._store, edges, self._tiles is not None)
                if mode == "tiles":
                    return mode, mode
            elif self._planes is not None and self.density >= MFMA_MIN_DENSITY and mfma_streamed(n, self.d_model, self.d_ff):
                return "mfma", "mfma"
            elif self._tiles is not None and pieces_us(n, self._store) < rows_us(n, self._store):
                return "tiles", "tiles"
        up = self.forced_up or up_mode(n, self.d_model)
        if up == "edges" and not edges:
            up = "rows"
        return up, self.forced_down or down_mode(n, self.d_ff)

    def forward(self, index: int, x: torch.Tensor) -> torch.Tensor:
        """y[N, d_model] of layer ``index`` for x[N, d_model] (contiguous float32 on the device).

        The result is a view of the runtime's output buffer, overwritten by the next call.
        """
        if x.dim() != 2 or x.shape[1] != self.d_model or x.dtype != torch.float32 or x.device != self._y.device or not x.is_contiguous():
            raise ValueError("expected a contiguous float32 [N, d_model] tensor on the runtime's device")
        n = x.shape[0]
        if not 1 <= n <= MAX_TOKENS:
            raise ValueError("unsupported token count")
        if n > self._tokens:
            self._reserve(n)
        up, down = self.modes(n)
        self._launch(index, x, n, up, down)
        self.calls[up, down] += 1
        return self._y[:n]

    def _tiles_args(self, index: int, y: int | None = None) -> tuple:
        """The arguments of ``hffn_forward_tiles`` / ``hffn_plan_tiles`` (or, for ``tiled=False``, of
        ``hffn_forward_tiles_compact`` / ``hffn_plan_tiles_compact``) between x and the widths; the output at ``y``
        (default: the start of the output buffer)."""
        tensors, tiles = self._tensors[index], self._tiles[index]
        _, act, _, y0 = self._work
        work = (act, self._tiles_work.data_ptr(), 4 * self._tiles_work.numel(), y0 if y is None else y)
        if not self.tiled:
            return (tensors["up_idx"].data_ptr(), tensors["up_val"].data_ptr(), tiles["up"].data_ptr(), tensors["b_up"].data_ptr(),
                    tensors["out_hidden"].data_ptr(), tensors["out_val"].data_ptr(), tiles["down"].data_ptr(),
                    tensors["b_down"].data_ptr(), *work)
        return (tiles["up"].data_ptr(), tiles["up_table"].data_ptr(), tensors["b_up"].data_ptr(), tiles["down"].data_ptr(),
                tiles["down_table"].data_ptr(), tensors["b_down"].data_ptr(), *work)

    def _tiles_forward(self, index: int, x: torch.Tensor, n: int, stream) -> None:
        """The tiles path on x (16-byte aligned), from the tiled store or the compact rows: one call per piece of up to
        ``TILES_MAX_TOKENS`` tokens (token-major rows of x and y, one after the other on the stream)."""
        entry = self._lib.hffn_forward_tiles if self.tiled else self._lib.hffn_forward_tiles_compact
        row = 4 * self.d_model  # bytes of one token's x or y
        for t0 in range(0, n, TILES_MAX_TOKENS):
            m = min(TILES_MAX_TOKENS, n - t0)
            _lib.check(entry(self._args[index][0], x.data_ptr() + row * t0, *self._tiles_args(index, self._y.data_ptr() + row * t0),
                             self.d_model, self.d_ff, *self._nnz[index], m, stream), "forward (tiles, tiles)")

    def _launch(self, index: int, x: torch.Tensor, n: int, up: str, down: str) -> None:
        value_type, *model = self._args[index]
        x_t, act, y_t, y = self._work
        stream = torch.cuda.current_stream(self.device).cuda_stream
        if up == "tiles":
            x = _aligned(x)  # read 16 bytes at a time
            self._fresh_tiles(index)
            self._tiles_forward(index, x, n, stream)
            return
        if up in PAIR_MODES:
            x = _aligned(x)  # the planes paths read x 16 bytes at a time
            if index in self._stale:
                self._densify(self._tensors[index], self._planes[index])
                self._stale.discard(index)
            planes, tensors = self._planes[index], self._tensors[index]
            if up == "gemv":
                _lib.check(self._lib.hffn_forward_gemv(value_type, x.data_ptr(), planes["up"].data_ptr(),
                                                       planes["up_binades"].data_ptr(), tensors["b_up"].data_ptr(),
                                                       planes["down"].data_ptr(), planes["down_binades"].data_ptr(),
                                                       tensors["b_down"].data_ptr(), act, self._gemv_work.data_ptr(),
                                                       4 * self._gemv_work.numel(), y, self.d_model, self.d_ff, n, stream),
                           "forward (gemv, gemv)")
                return
            _lib.check(self._lib.hffn_forward_mfma(value_type, x.data_ptr(), planes["up"].data_ptr(),
                                                   planes["up_binades"].data_ptr(), tensors["b_up"].data_ptr(),
                                                   planes["down"].data_ptr(), planes["down_binades"].data_ptr(),
                                                   tensors["b_down"].data_ptr(), self._mfma_work.data_ptr(),
                                                   4 * self._mfma_work.numel(), y,
                                                   self.d_model, self.d_ff, n, stream), "forward (mfma, mfma)")
            return
        _lib.check(self._lib.hffn_forward(_lib.UP_MODES[up], _lib.DOWN_MODES[down], value_type, x.data_ptr(), *model,
                                          x_t, act, y_t, y, self.d_model, self.d_ff, *self._nnz[index], n, leading_dim(n),
                                          stream),
                   f"forward ({up}, {down})")
