"""One training step of an HFFN layer on the HIP library: the forward with the pre-activations kept, the backward and a
compact AdamW, over an inference ``HFFNRuntime`` whose compact arrays and work buffers it reads and updates in place.

Interface of ``HFFNTrainRuntime`` (``runtime/gpu/nvidia/ffn/training/train_runtime.py:61-247``, kernels
``kernels_train.py:101-258``): the constructor ``(runtime, lr, betas, eps, weight_decay, max_tokens)``, ``reserve``,
``forward(index, x, z=None)``, ``backward(index, gy)``, ``adamw(index)``, ``step(index, x, gy)``, the views
``parameters/gradients/moments/supports/activations``, ``nbytes``, and the counters ``steps``, ``calls`` and
``growths``. Gradients and moments keep the order of their arrays (``out_val`` output-major, as the runtime holds it);
no dense weight, gradient or moment exists.

State kept per layer (``_LayerState``): gradients and AdamW moments of ``up_val``, ``b_up``, ``out_val``, ``b_down``;
the two transposed supports, built on the device by the library's stable counting sort with the slot positions as the
payload (``hffn_output_major``): up slots by input feature (``in_offsets``, ``in_hidden`` = owner neuron, ``in_pos`` =
position in ``up_val``) and down edges by neuron (``hid_offsets``, ``hid_output`` = output feature, ``hid_pos`` =
position in ``out_val``); the values in those two orders (gathered from the compact arrays at every backward); and the
layer's columns in the shared partial workspace. Shared by the layers and sized by ``reserve``: ``z``, ``gz``
``[d_ff, ld]``, ``gy_t``, ``gx_t`` ``[d_model, ld]``, ``gx`` ``[N, d_model]`` (``ld = leading_dim(N)``), the token-tile
partials ``[tiles, columns]`` of the gather sampled products, and the workspace of the dense sampled products.

The step: ``hffn_forward_z`` (the runtime's gather forward writing ``z``); the sampled products ``g_down``/``gb_down``
and ``g_up``/``gb_up`` as gathers over 256-token tiles (``hffn_grad_sddmm``, tiles added in order by
``hffn_reduce_tiles``) or, from ``GRAD_DENSE_MIN_TOKENS`` tokens on dense enough layers, as split-fp16 MFMA products
sampled at the support (``hffn_grad_dense``); ``gz`` by ``hffn_grad_hidden``; ``gx`` by ``hffn_grad_x``; AdamW per
array by ``hffn_adamw``. After an update the runtime's densified planes of that layer are rebuilt before their next use.
On layers whose runtime holds densified planes, from ``TRAIN_MFMA_MIN_TOKENS`` tokens (``train_mode``), the forward
with z (``hffn_forward_mfma_z``) and gz, gx (``hffn_backward_mfma``) run as split-fp16 MFMA products instead, the
backward over planes of W_down^T and W_up^T densified at every backward from the values in the transposed orders.
"""
from __future__ import annotations

import ctypes
import math
from collections import Counter
from dataclasses import dataclass

import torch

from . import _lib
from .runtime import MAX_TOKENS, PAIR_MODES, HFFNRuntime, _aligned, down_mode, edges_supported, leading_dim, mfma_streamed, up_mode

PARAMETERS = ("up_val", "b_up", "out_val", "b_down")
SUPPORTS = ("in_offsets", "in_pos", "in_hidden", "hid_offsets", "hid_pos", "hid_output")
GRAD_TILE = 256              # tokens per tile of the gather sampled products
PARTIAL_MAX_TOKENS = 2048    # tokens the tile partials are sized for at construction
GRAD_DENSE_MIN_TOKENS = 64   # from this N the sampled products may run as dense MFMA products
GRAD_DENSE_MIN_DENSITY = 0.05  # on layers of at least this support density (the products' dense work over the useful)
GRAD_MODES = ("gather", "dense")
TRAIN_MFMA_MIN_TOKENS = 64   # from this N the forward with z, gz and gx may run on the planes
TRAIN_MODES = ("gather", "mfma")


def grad_tiles(n: int) -> int:
    """Token tiles of the gather sampled products for N tokens (1: no partials, no reduction)."""
    return -(-n // GRAD_TILE)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def group_by_index(offsets: torch.Tensor, index: torch.Tensor, rows: int, bins: int) -> dict[str, torch.Tensor]:
    """The slots of a row-major support (``offsets`` int32[rows + 1], ``index`` int16 in [0, bins)) regrouped by index,
    stably (slot order kept within an index), on the device: ``offsets`` int32[bins + 1], ``owner`` int16 (the row of
    each slot) and ``position`` int32 (the slot's place in the row-major arrays). The library's counting sort moves
    32-bit payloads without arithmetic, so the positions travel as its value payload."""
    lib = _lib.load()
    device = index.device
    nnz = index.numel()
    positions = torch.arange(nnz, dtype=torch.int32, device=device)
    grouped = {"offsets": torch.empty(bins + 1, dtype=torch.int32, device=device),
               "owner": torch.empty(nnz, dtype=torch.int16, device=device),
               "position": torch.empty(nnz, dtype=torch.int32, device=device)}
    work = torch.empty(max(4, _lib.query_bytes(lib.hffn_output_major_workspace, nnz, bins)), dtype=torch.uint8, device=device)
    _lib.check(lib.hffn_output_major(_lib.VALUE_F32, offsets.data_ptr(), index.data_ptr(), positions.data_ptr(), bins, rows, nnz,
                                     grouped["offsets"].data_ptr(), grouped["owner"].data_ptr(), grouped["position"].data_ptr(),
                                     work.data_ptr(), work.numel(), _stream(device)), "regroup by index")
    torch.cuda.current_stream(device).synchronize()  # `positions` and `work` are released on return
    return grouped


@dataclass
class _LayerState:
    grads: dict
    moments: dict
    supports: dict
    values: dict          # in_val, hid_val: the compact values in the transposed orders
    columns: tuple        # g_down [0, c1), gb_down [c1, c2), g_up [c2, c3), gb_up [c3, width) of the partials
    planes_t: dict | None = None  # planes of W_down^T and W_up^T (the MFMA backward), allocated by reserve


class HFFNTrainRuntime:
    """Training step over an ``HFFNRuntime`` of fp32 layers (see the module docstring)."""

    def __init__(self, runtime: HFFNRuntime, lr: float = 1e-3, betas: tuple[float, float] = (0.9, 0.999),
                 eps: float = 1e-8, weight_decay: float = 1e-2, max_tokens: int = PARTIAL_MAX_TOKENS) -> None:
        self.runtime = runtime
        self.d_model, self.d_ff = runtime.d_model, runtime.d_ff
        self.lr, self.betas, self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self._lib = _lib.load()
        self._layers = [self._layer_state(arrays) for arrays in runtime._tensors]
        self.steps = [0] * len(self._layers)   # AdamW steps taken per layer
        self.calls: Counter = Counter()        # (up, down) of the forwards that kept z
        self.forced_grad: str | None = None    # diagnostic: the sampled products' formulation, else the policy's
        self.forced_train: str | None = None   # diagnostic: the forward with z, gz and gx on gathers or planes
        self._mfma_work: torch.Tensor | None = None
        self._tokens = 0                        # N the dense buffers hold
        self._tiles = 1                         # token tiles the partials hold (none allocated for 1)
        self._partials: torch.Tensor | None = None
        self._dense_work: torch.Tensor | None = None
        self._last_forward: tuple | None = None  # (index, n, z pointer, runtime calls) of the last forward with z
        self.growths = 0
        self.reserve(1)
        self._grow_partials(max_tokens)
        self._grow_dense(max_tokens)
        self.growths = 0                        # growths after construction: a timed window must see none

    def _layer_state(self, arrays: dict) -> _LayerState:
        if arrays["up_val"].dtype != torch.float32:
            raise ValueError("the training step updates float32 values; this layer holds "
                             f"{arrays['up_val'].dtype}")
        for offsets, values in (("up_offsets", "up_val"), ("out_offsets", "out_val")):
            if int(arrays[offsets][0]) != 0 or int(arrays[offsets][-1]) != arrays[values].numel():
                raise ValueError(f"{offsets} must start at 0 and end at the length of {values}: every slot owns one "
                                 "partial column")
        by_input = group_by_index(arrays["up_offsets"], arrays["up_idx"], self.d_ff, self.d_model)
        by_neuron = group_by_index(arrays["out_offsets"], arrays["out_hidden"], self.d_model, self.d_ff)
        supports = {"in_offsets": by_input["offsets"], "in_pos": by_input["position"], "in_hidden": by_input["owner"],
                    "hid_offsets": by_neuron["offsets"], "hid_pos": by_neuron["position"], "hid_output": by_neuron["owner"]}
        c1 = arrays["out_val"].numel()
        c2 = c1 + self.d_model
        c3 = c2 + arrays["up_val"].numel()
        return _LayerState(grads={name: torch.zeros_like(arrays[name]) for name in PARAMETERS},
                           moments={name: (torch.zeros_like(arrays[name]), torch.zeros_like(arrays[name])) for name in PARAMETERS},
                           supports=supports,
                           values={"in_val": torch.empty_like(arrays["up_val"]), "hid_val": torch.empty_like(arrays["out_val"])},
                           columns=(c1, c2, c3, c3 + self.d_ff))

    # -- buffers ---------------------------------------------------------------------------------------------------
    def reserve(self, n: int) -> None:
        """Size every buffer of a step on N tokens; allocates only what must grow (counted in ``growths``)."""
        runtime = self.runtime
        if n > runtime._tokens:
            runtime._reserve(n)
            self._last_forward = None
            self.growths += 1
        if n > self._tokens:
            ld = leading_dim(n)
            device = runtime.device
            self._z, self._gz = (torch.empty(self.d_ff * ld, device=device) for _ in range(2))
            self._gy_t, self._gx_t = (torch.empty(self.d_model * ld, device=device) for _ in range(2))
            self._gx = torch.empty(n, self.d_model, device=device)
            self._tokens = n
            self._last_forward = None
            self.growths += 1
        self._grow_partials(n)
        self._grow_dense(n)
        self._grow_mfma(n)

    def _mfma_possible(self, n: int) -> bool:
        return self.runtime.mfma_available and mfma_streamed(n, self.d_model, self.d_ff)

    def _grow_mfma(self, n: int) -> None:
        """The MFMA workspace at N and every layer's transposed planes, when the planes products may run at N."""
        if not self._mfma_possible(n):
            return
        need = _lib.query_bytes(self._lib.hffn_train_mfma_workspace, n, self.d_model, self.d_ff)
        if self._mfma_work is None or need > self._mfma_work.numel():
            self._mfma_work = torch.zeros(need, dtype=torch.uint8, device=self.runtime.device)
            self.growths += 1
        for state in self._layers:
            if state.planes_t is None:
                device, planes = self.runtime.device, {}
                for side, rows, k in (("down_t", self.d_ff, self.d_model), ("up_t", self.d_model, self.d_ff)):
                    size = _lib.query_bytes(self._lib.hffn_dense_planes_bytes, rows, k)
                    planes[side] = torch.empty(size // 2, dtype=torch.float16, device=device)
                    planes[f"{side}_binades"] = torch.empty(rows, dtype=torch.int32, device=device)
                state.planes_t = planes
                self.growths += 1

    def _grow_partials(self, n: int) -> None:
        tiles = grad_tiles(n)
        if tiles <= self._tiles:
            return
        width = max(state.columns[3] for state in self._layers)
        if tiles * width >= 1 << 32:
            raise ValueError(f"{tiles} token tiles x {width} partial columns do not fit the kernels' 32-bit offsets")
        self._partials = torch.empty(tiles * width, device=self.runtime.device)
        self._tiles = tiles
        self.growths += 1

    def _dense_bytes_at(self, n: int) -> int:
        """Workspace bytes of the dense sampled products at N (both shapes), 0 if the streamed GEMM refuses either."""
        need = 0
        for rows, cols in ((self.d_model, self.d_ff), (self.d_ff, self.d_model)):
            size = ctypes.c_uint64(0)
            if self._lib.hffn_grad_dense_workspace(rows, cols, n, ctypes.byref(size)) != _lib.OK:
                return 0
            need = max(need, size.value)
        return need

    def _grow_dense(self, n: int) -> None:
        if self.grad_mode(n) != "dense":
            return
        need = self._dense_bytes_at(n)
        if self._dense_work is None or need > self._dense_work.numel():
            self._dense_work = torch.empty(need, dtype=torch.uint8, device=self.runtime.device)
            self.growths += 1

    def grad_mode(self, n: int) -> str:
        """``dense`` (MFMA products over the tokens, sampled at the support) from ``GRAD_DENSE_MIN_TOKENS`` tokens on
        layers of at least ``GRAD_DENSE_MIN_DENSITY`` whose shapes the streamed GEMM takes, else ``gather``;
        ``forced_grad`` overrides the choice."""
        if self.forced_grad is not None:
            if self.forced_grad not in GRAD_MODES:
                raise ValueError(f"sampled-product mode is one of {GRAD_MODES}, not {self.forced_grad!r}")
            if self.forced_grad == "dense" and not self._dense_bytes_at(n):
                raise ValueError(f"the dense sampled products do not run at N={n} on {self.d_model} x {self.d_ff}")
            return self.forced_grad
        dense = n >= GRAD_DENSE_MIN_TOKENS and self.runtime.density >= GRAD_DENSE_MIN_DENSITY and self._dense_bytes_at(n) > 0
        return "dense" if dense else "gather"

    def train_mode(self, n: int) -> str:
        """``mfma`` (the forward with z, gz and gx as split-fp16 MFMA products over densified planes) from
        ``TRAIN_MFMA_MIN_TOKENS`` tokens when the runtime holds planes, runs its policy (no forced pair) and the streamed
        GEMM takes N, else ``gather``; ``forced_train`` overrides the choice."""
        possible = self._mfma_possible(n)
        if self.forced_train is not None:
            if self.forced_train not in TRAIN_MODES:
                raise ValueError(f"training mode is one of {TRAIN_MODES}, not {self.forced_train!r}")
            if self.forced_train == "mfma" and not possible:
                raise ValueError(f"the planes products do not run at N={n} on {self.d_model} x {self.d_ff} (no planes, or "
                                 "a shape the streamed GEMM refuses)")
            return self.forced_train
        policy = self.runtime.forced_up is None and self.runtime.forced_down is None
        return "mfma" if possible and policy and n >= TRAIN_MFMA_MIN_TOKENS else "gather"

    def _runtime_planes(self, index: int) -> dict:
        """The runtime's planes of layer ``index``, rebuilt first if an update made them stale."""
        runtime = self.runtime
        if index in runtime._stale:
            runtime._densify(runtime._tensors[index], runtime._planes[index])
            runtime._stale.discard(index)
        return runtime._planes[index]

    def _tokens_of(self, t: torch.Tensor, name: str) -> int:
        if not (t.dim() == 2 and t.shape[1] == self.d_model and t.dtype == torch.float32 and t.device == self.runtime._y.device
                and t.is_contiguous()):
            raise ValueError(f"{name}: a contiguous float32 [N, {self.d_model}] tensor on {self.runtime._y.device} is required")
        if not 1 <= t.shape[0] <= MAX_TOKENS:
            raise ValueError(f"{name}: N={t.shape[0]} outside [1, {MAX_TOKENS}]")
        return t.shape[0]

    def modes(self, n: int) -> tuple[str, str]:
        """The gather kernels a forward with z runs: the runtime's forced pair, else its gather policy (the planes paths
        keep no float32 activations)."""
        runtime = self.runtime
        if runtime.forced_up in PAIR_MODES:
            raise ValueError(f"a forward that keeps z runs the gather kernels; the runtime is forced to {runtime.forced_up}")
        up = runtime.forced_up or up_mode(n, self.d_model)
        if up == "edges" and not edges_supported(self.d_model, n):
            up = "rows"
        return up, runtime.forced_down or down_mode(n, self.d_ff)

    # -- the step ----------------------------------------------------------------------------------------------------
    def forward(self, index: int, x: torch.Tensor, z: torch.Tensor | None = None) -> torch.Tensor:
        """y [N, d_model] of layer ``index`` (a view of the runtime's output buffer). Without ``z`` this is the inference
        call itself. With ``z`` (contiguous float32 on the device, ``d_ff * leading_dim(N)`` entries or more) the gather
        forward also writes the pre-activations there, hidden-major ``[d_ff, leading_dim(N)]``, and remembers what the
        backward of this layer needs; ``z`` must live until then."""
        runtime = self.runtime
        if z is None:
            return runtime.forward(index, x)
        n = self._tokens_of(x, "x")
        ld = leading_dim(n)
        if not (z.dtype == torch.float32 and z.device == runtime._y.device and z.is_contiguous() and z.numel() >= self.d_ff * ld):
            raise ValueError(f"z must be a contiguous float32 device tensor of at least {self.d_ff * ld} entries")
        self.reserve(n)
        x_t, act, y_t, y = runtime._work
        if self.train_mode(n) == "mfma":
            planes, tensors, x = self._runtime_planes(index), runtime._tensors[index], _aligned(x)
            _lib.check(self._lib.hffn_forward_mfma_z(x.data_ptr(), planes["up"].data_ptr(), planes["up_binades"].data_ptr(),
                                                     tensors["b_up"].data_ptr(), planes["down"].data_ptr(),
                                                     planes["down_binades"].data_ptr(), tensors["b_down"].data_ptr(),
                                                     self._mfma_work.data_ptr(), self._mfma_work.numel(), x_t, act, z.data_ptr(),
                                                     y, self.d_model, self.d_ff, n, ld, _stream(runtime.device)),
                       "forward with z (mfma)")
            self.calls["mfma", "mfma"] += 1
        else:
            up, down = self.modes(n)
            _, *model = runtime._args[index]
            _lib.check(self._lib.hffn_forward_z(_lib.UP_MODES[up], _lib.DOWN_MODES[down], x.data_ptr(), *model, x_t, act, y_t, y,
                                                z.data_ptr(), self.d_model, self.d_ff, *runtime._nnz[index], n, ld,
                                                _stream(runtime.device)), f"forward with z ({up}, {down})")
            self.calls[up, down] += 1
        self._last_forward = (index, n, z.data_ptr(), sum(runtime.calls.values()))
        return runtime._y[:n]

    def backward(self, index: int, gy: torch.Tensor) -> torch.Tensor:
        """The compact gradients of layer ``index`` (``gradients(index)``) and gx [N, d_model] (a view of the step's buffer)
        for gy [N, d_model], from the state of the last forward with z."""
        runtime = self.runtime
        last = self._last_forward
        if last is None or last[0] != index or last[3] != sum(runtime.calls.values()):
            raise RuntimeError(f"backward({index}) must follow forward({index}, x, z) directly; another forward ran in "
                               "between, or none kept z")
        _, n, z_ptr, _ = last
        if self._tokens_of(gy, "gy") != n:
            raise ValueError(f"gy has {gy.shape[0]} tokens; it must have the N of the forward ({n})")
        lib, stream, ld, d, h = self._lib, _stream(runtime.device), leading_dim(n), self.d_model, self.d_ff
        arrays, state = runtime._tensors[index], self._layers[index]
        supports, values, grads = state.supports, state.values, state.grads
        x_t, act, _, _ = runtime._work
        _lib.check(lib.hffn_transpose(gy.data_ptr(), self._gy_t.data_ptr(), n, d, d, ld, stream), "gy feature-major")
        for source, position, target in (("out_val", "hid_pos", "hid_val"), ("up_val", "in_pos", "in_val")):
            _lib.check(lib.hffn_gather_values(arrays[source].data_ptr(), supports[position].data_ptr(), values[target].data_ptr(),
                                              values[target].numel(), stream), f"{target} refresh")
        planes_mode = self.train_mode(n) == "mfma"
        if planes_mode:  # gz and gx on the planes of W_down^T and W_up^T, densified from the values just gathered
            planes_t = state.planes_t
            for side, rows, k, (offsets, owner, vals) in (("down_t", h, d, ("hid_offsets", "hid_output", "hid_val")),
                                                          ("up_t", d, h, ("in_offsets", "in_hidden", "in_val"))):
                source = values[vals]
                _lib.check(lib.hffn_densify(_lib.VALUE_F32, supports[offsets].data_ptr(), supports[owner].data_ptr(),
                                            source.data_ptr(), rows, k, planes_t[side].data_ptr(),
                                            planes_t[f"{side}_binades"].data_ptr(), stream), f"densify {side}")
            gy_in = _aligned(gy)
            _lib.check(lib.hffn_backward_mfma(gy_in.data_ptr(), z_ptr, planes_t["down_t"].data_ptr(),
                                              planes_t["down_t_binades"].data_ptr(), planes_t["up_t"].data_ptr(),
                                              planes_t["up_t_binades"].data_ptr(), self._mfma_work.data_ptr(),
                                              self._mfma_work.numel(), self._gz.data_ptr(), self._gx.data_ptr(), d, h, n, ld, stream),
                       "gz, gx (mfma)")
        dense = self.grad_mode(n) == "dense"
        if dense:
            self._grow_dense(n)
        c1, c2, c3, width = state.columns
        tiled = not dense and grad_tiles(n) > 1
        if tiled:  # tile partials in the shared workspace, added in tile order below
            base = self._partials.data_ptr()
            into = {"g_down": base, "gb_down": base + 4 * c1, "g_up": base + 4 * c2, "gb_up": base + 4 * c3}
        else:      # one tile, or the dense products: straight into the gradients
            into = {"g_down": grads["out_val"].data_ptr(), "gb_down": grads["b_down"].data_ptr(),
                    "g_up": grads["up_val"].data_ptr(), "gb_up": grads["b_up"].data_ptr()}
        stride = width if tiled else 0

        def sampled(row, mat, owner_offsets, owner_index, g, gb, rows, cols, what):
            if dense:
                _lib.check(lib.hffn_grad_dense(row, mat, owner_offsets, owner_index, g, gb, rows, cols, n, ld,
                                               self._dense_work.data_ptr(), self._dense_work.numel(), stream), f"{what} (dense)")
            else:
                _lib.check(lib.hffn_grad_sddmm(row, mat, owner_offsets, owner_index, g, gb, rows, n, ld, stride, stream), what)

        sampled(self._gy_t.data_ptr(), act, arrays["out_offsets"].data_ptr(), arrays["out_hidden"].data_ptr(), into["g_down"],
                into["gb_down"], d, h, "g_down")
        if not planes_mode:
            _lib.check(lib.hffn_grad_hidden(gy.data_ptr(), self._gy_t.data_ptr(), z_ptr, supports["hid_offsets"].data_ptr(),
                                            supports["hid_output"].data_ptr(), values["hid_val"].data_ptr(), self._gz.data_ptr(), d, h,
                                            values["hid_val"].numel(), n, ld, stream), "gz")
        sampled(self._gz.data_ptr(), x_t, arrays["up_offsets"].data_ptr(), arrays["up_idx"].data_ptr(), into["g_up"], into["gb_up"],
                h, d, "g_up")
        if tiled:
            _lib.check(lib.hffn_reduce_tiles(self._partials.data_ptr(), width, grad_tiles(n), c1, c2, c3,
                                             grads["out_val"].data_ptr(), grads["b_down"].data_ptr(), grads["up_val"].data_ptr(),
                                             grads["b_up"].data_ptr(), stream), "tile partials")
        if not planes_mode:
            _lib.check(lib.hffn_grad_x(self._gz.data_ptr(), supports["in_offsets"].data_ptr(), supports["in_hidden"].data_ptr(),
                                       values["in_val"].data_ptr(), self._gx_t.data_ptr(), self._gx.data_ptr(), d, h,
                                       values["in_val"].numel(), n, ld, stream), "gx")
        return self._gx[:n]

    def adamw(self, index: int) -> None:
        """One AdamW update of the four arrays of layer ``index`` from its last gradients (decoupled decay, bias
        corrections computed in float64 on the host)."""
        self.steps[index] += 1
        k = self.steps[index]
        beta1, beta2 = self.betas
        scalars = (self.lr * self.weight_decay, beta1, 1.0 - beta1, beta2, 1.0 - beta2, self.lr / (1.0 - beta1 ** k),
                   math.sqrt(1.0 - beta2 ** k), self.eps)
        arrays, state = self.runtime._tensors[index], self._layers[index]
        stream = _stream(self.runtime.device)
        for name in PARAMETERS:
            first, second = state.moments[name]
            _lib.check(self._lib.hffn_adamw(arrays[name].data_ptr(), state.grads[name].data_ptr(), first.data_ptr(),
                                            second.data_ptr(), arrays[name].numel(), *scalars, stream), f"AdamW of {name}")
        self.runtime.invalidate_planes(index)

    def step(self, index: int, x: torch.Tensor, gy: torch.Tensor) -> torch.Tensor:
        """Forward (z in the step's own buffer), backward and AdamW of layer ``index``; returns gx (a view)."""
        self.reserve(self._tokens_of(x, "x"))
        self.forward(index, x, self._z)
        gx = self.backward(index, gy)
        self.adamw(index)
        return gx

    # -- views (no copies) -------------------------------------------------------------------------------------------
    def parameters(self, index: int) -> dict[str, torch.Tensor]:
        return {name: self.runtime._tensors[index][name] for name in PARAMETERS}

    def gradients(self, index: int) -> dict[str, torch.Tensor]:
        """By parameter, in the order of the parameter's array (``out_val``: output-major edges)."""
        return self._layers[index].grads

    def moments(self, index: int) -> dict[str, tuple[torch.Tensor, torch.Tensor]]:
        return self._layers[index].moments

    def supports(self, index: int) -> dict[str, torch.Tensor]:
        return self._layers[index].supports

    def activations(self, n: int) -> dict[str, torch.Tensor]:
        """z, h and gz hidden-major [d_ff, N] (strided views of the [d_ff, leading_dim(N)] buffers) and gx [N, d_model]
        of the last step on N tokens."""
        ld = leading_dim(n)
        view = lambda buffer: buffer[:self.d_ff * ld].view(self.d_ff, ld)[:, :n]  # noqa: E731
        return {"z": view(self._z), "h": view(self.runtime._act), "gz": view(self._gz), "gx": self._gx[:n]}

    def nbytes(self, index: int) -> dict[str, int]:
        """Bytes held for layer ``index``: its values, gradients, moments, indices (the runtime's, the transposed supports
        and the values in their orders), the shared dense workspace and the shared tile partials."""
        size = lambda tensors: sum(t.numel() * t.element_size() for t in tensors)  # noqa: E731
        arrays, state = self.runtime._tensors[index], self._layers[index]
        return {"values": size(arrays[name] for name in PARAMETERS),
                "gradients": size(state.grads.values()),
                "moments": size(t for pair in state.moments.values() for t in pair),
                "indices": size(arrays[name] for name in ("up_offsets", "up_idx", "out_offsets", "out_hidden"))
                + size(state.supports.values()) + size(state.values.values()),
                "workspace": self.runtime.workspace_bytes() + size((self._z, self._gz, self._gy_t, self._gx_t, self._gx))
                + (self._dense_work.numel() if self._dense_work is not None else 0)
                + (self._mfma_work.numel() if self._mfma_work is not None else 0),
                "planes_t": size(state.planes_t.values()) if state.planes_t is not None else 0,
                "partials": size((self._partials,)) if self._partials is not None else 0}
