"""``HFFNTrainRuntime``: one training step of an HFFN layer (forward with the pre-activations kept, backward, compact
AdamW) over the inference runtime, as ``train_runtime.HFFNTrainRuntime`` of
``runtime/gpu/nvidia/ffn/training/train_runtime.py:61-247`` (kernels: ``kernels_train.py:101-258``).

The wrapped ``HFFNRuntime`` keeps its compact arrays and work buffers (``x_t``, ``act = h``, ``y``); the step reads
and updates them in place. Added here, allocated at construction or by ``reserve(n)``:

* per layer: the gradients of ``up_val``, ``b_up``, ``out_val``, ``b_down`` and their two AdamW moments, each of the
  length and order of its array (``out_val`` output-major, as the runtime holds it); the two transposed supports as
  positions into the runtime's arrays (up slots input-major: ``in_offsets``, ``in_pos``, ``in_hidden``; down edges
  hidden-major: ``hid_offsets``, ``hid_pos``, ``hid_output``), and the values in those orders, refreshed from the
  compact arrays by a device gather at each backward;
* dense, shared by the layers: ``z``, ``gz`` ``[d_ff, ld]``, ``gy_t``, ``gx_t`` ``[d_model, ld]``, ``gx`` ``[N, d_model]``
  (``ld = leading_dim(N)``, the runtime's stride);
* the tile partials of the two sampled products, ``[tiles, S]`` with ``S = nnz_down + d_model + nnz_up + d_ff``
  columns, sized at construction for ``max_tokens`` and grown only by ``reserve``;
* for the dense sampled products (from ``GRAD_DENSE_MIN_TOKENS`` tokens): the planes of both operands over the tokens
  and the GEMM's partials (``hffn_grad_dense_workspace``), sized like the tile partials.

No dense ``W_up``, ``W_down``, gradient or moment exists. The kernels: the forward is the runtime's gather forward with
``z`` stored (``hffn_forward_z``); ``g_down``/``gb_down`` and ``g_up``/``gb_up`` are sampled products
(``hffn_grad_sddmm``) over token tiles of 256, summed in tile order (``hffn_reduce_tiles``) above 256 tokens, or from
64 tokens dense split-fp16 MFMA products gathered at the support (``hffn_grad_dense``, ``grad_mode``); ``gz`` is
the rows up kernel over the hidden-major down support with a gelu' epilogue (``hffn_grad_hidden``); ``gx`` the rows
down kernel over the input-major up support (``hffn_grad_x``); AdamW elementwise (``hffn_adamw``). fp32 values only.

``backward(index, gy)`` uses the state of the last ``forward(index, x, z)`` with a ``z`` buffer and must follow it with
no other forward of the runtime in between (checked). After an update the runtime's densified planes (its MFMA path)
of that layer are rebuilt before their next use.
"""
from __future__ import annotations

import math
from collections import Counter

import torch

from . import _lib
from .runtime import MAX_TOKENS, MFMA_MIN_DENSITY, HFFNRuntime, down_mode, edges_supported, leading_dim, up_mode

PARAMETERS = ("up_val", "b_up", "out_val", "b_down")
SUPPORTS = ("in_offsets", "in_pos", "in_hidden", "hid_offsets", "hid_pos", "hid_output")
GRAD_TILE = 256              # tokens per tile of the sampled products
PARTIAL_MAX_TOKENS = 2048    # default largest N: the tile partials are sized at construction, never in a step
GRAD_DENSE_MIN_TOKENS = 64   # from this N the sampled products run as dense MFMA products (when the shapes allow)
GRAD_MODES = ("gather", "dense")


def grad_tiles(n: int) -> int:
    """Token tiles of the sampled products for N tokens; 1 means no partials and no reduction launch."""
    return (n + GRAD_TILE - 1) // GRAD_TILE


def transposed_supports(layer) -> dict[str, torch.Tensor]:
    """Up slots input-major and down edges hidden-major, as positions into the runtime's arrays (load time, host).

    Stable orders: the up slots of one input in ascending hidden order, the down edges of one neuron in ascending
    output order (``train_runtime.py:41-58``); these are the summation orders of ``gx`` and ``gz``."""
    up_offsets, up_idx = layer.up_offsets.cpu().long(), layer.up_idx.cpu().long()
    out_offsets, out_hidden = layer.out_offsets.cpu().long(), layer.out_hidden.cpu().long()
    up_hidden = torch.repeat_interleave(torch.arange(layer.d_ff), up_offsets.diff())
    by_input = torch.argsort(up_idx, stable=True)
    in_offsets = torch.zeros(layer.d_model + 1, dtype=torch.int32)
    in_offsets[1:] = torch.cumsum(torch.bincount(up_idx, minlength=layer.d_model), 0)
    out_output = torch.repeat_interleave(torch.arange(layer.d_model), out_offsets.diff())
    by_hidden = torch.argsort(out_hidden, stable=True)
    hid_offsets = torch.zeros(layer.d_ff + 1, dtype=torch.int32)
    hid_offsets[1:] = torch.cumsum(torch.bincount(out_hidden, minlength=layer.d_ff), 0)
    return {"in_offsets": in_offsets, "in_pos": by_input.to(torch.int32), "in_hidden": up_hidden[by_input].to(torch.int16),
            "hid_offsets": hid_offsets, "hid_pos": by_hidden.to(torch.int32), "hid_output": out_output[by_hidden].to(torch.int16)}


class HFFNTrainRuntime:
    def __init__(self, runtime: HFFNRuntime, lr: float = 1e-3, betas: tuple[float, float] = (0.9, 0.999),
                 eps: float = 1e-8, weight_decay: float = 1e-2, max_tokens: int = PARTIAL_MAX_TOKENS) -> None:
        self.runtime = runtime
        self.d_model, self.d_ff = runtime.d_model, runtime.d_ff
        self.lr, self.betas, self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self._lib = _lib.load()
        device = runtime.device
        self._supports, self._grads, self._moments, self._transposed_values = [], [], [], []
        self._columns = []
        for layer, params in zip(runtime.layers, runtime._tensors):
            if params["up_val"].dtype != torch.float32:
                raise ValueError("training needs float32 values")
            for offsets, values in (("out_offsets", "out_val"), ("up_offsets", "up_val")):
                if int(params[offsets][0]) != 0 or int(params[offsets][-1]) != params[values].numel():
                    raise ValueError(f"{offsets} must cover {values} exactly (partial workspace columns)")
            supports = {name: t.to(device) for name, t in transposed_supports(layer).items()}
            self._supports.append(supports)
            self._grads.append({name: torch.zeros_like(params[name]) for name in PARAMETERS})
            self._moments.append({name: (torch.zeros_like(params[name]), torch.zeros_like(params[name])) for name in PARAMETERS})
            self._transposed_values.append({"in_val": torch.empty_like(params["up_val"]),
                                            "hid_val": torch.empty_like(params["out_val"])})
            c1 = params["out_val"].numel()
            c2 = c1 + self.d_model
            c3 = c2 + params["up_val"].numel()
            self._columns.append((c1, c2, c3, c3 + self.d_ff))
        self.steps = [0] * len(runtime.layers)   # AdamW step count per layer (part of the optimiser state)
        self.calls: Counter = Counter()          # (up, down) of the forwards with a z buffer
        self._partial_tiles, self._partials = 1, None
        self._dense_bytes, self._dense_work = 0, None
        self.forced_grad: str | None = None      # diagnostic: fix the sampled products' formulation
        self._saved: tuple | None = None
        self._tokens = 0
        self.growths = 0
        self.reserve(1)
        self._reserve_partials(max_tokens)
        self._reserve_dense(max_tokens)
        self.growths = 0     # buffer growths after construction: a timed window must leave it unchanged

    # -- buffers ---------------------------------------------------------------------------------------------------
    def reserve(self, n: int) -> None:
        """Size the runtime's and the step's buffers for N tokens. Allocates only when N grows."""
        runtime = self.runtime
        if n > runtime._tokens:
            runtime._reserve(n)
            self._saved = None
            self.growths += 1
        if n > self._tokens:
            self._tokens = n
            self.growths += 1
            device, ld = runtime.device, leading_dim(n)
            self._z = torch.empty(self.d_ff * ld, device=device)
            self._gz = torch.empty(self.d_ff * ld, device=device)
            self._gy_t = torch.empty(self.d_model * ld, device=device)
            self._gx_t = torch.empty(self.d_model * ld, device=device)
            self._gx = torch.empty(n, self.d_model, device=device)
            self._saved = None
        self._reserve_partials(n)
        self._reserve_dense(n)

    def _dense_need(self, n: int) -> int:
        """Workspace bytes of the dense sampled products at N (the larger of the two shapes), 0 where the streamed GEMM
        does not take them."""
        need = 0
        for rows, cols in ((self.d_model, self.d_ff), (self.d_ff, self.d_model)):
            result = _lib.ctypes.c_uint64(0)
            if self._lib.hffn_grad_dense_workspace(rows, cols, n, _lib.ctypes.byref(result)) != _lib.OK:
                return 0
            need = max(need, result.value)
        return need

    def _reserve_dense(self, n: int) -> None:
        if self.grad_mode(n) != "dense":
            return
        need = self._dense_need(n)
        if need > self._dense_bytes:
            self._dense_bytes = need
            self.growths += 1
            self._dense_work = torch.empty(need, dtype=torch.uint8, device=self.runtime.device)

    def grad_mode(self, n: int) -> str:
        """How the two sampled products run at N: ``dense`` (split-fp16 MFMA products over the tokens, then the
        support's entries) from ``GRAD_DENSE_MIN_TOKENS`` on layers of at least ``MFMA_MIN_DENSITY`` whose shapes the
        streamed GEMM takes; else ``gather`` (``hffn_grad_sddmm``). ``forced_grad`` overrides it."""
        if self.forced_grad is not None:
            if self.forced_grad not in GRAD_MODES:
                raise ValueError("unknown sampled-product mode")
            if self.forced_grad == "dense" and self._dense_need(n) == 0:
                raise ValueError("the dense sampled products do not take this shape")
            return self.forced_grad
        if n >= GRAD_DENSE_MIN_TOKENS and self.runtime.density >= MFMA_MIN_DENSITY and self._dense_need(n) > 0:
            return "dense"
        return "gather"

    def _reserve_partials(self, n: int) -> None:
        tiles = grad_tiles(n)
        if tiles <= self._partial_tiles:
            return
        stride = max(columns[3] for columns in self._columns)
        if tiles * stride >= 2 ** 32:      # the kernels address the workspace with unsigned 32-bit indices
            raise ValueError(f"partial workspace of {tiles} tiles x {stride} columns exceeds 32-bit indexing")
        self._partial_tiles = tiles
        self.growths += 1
        self._partials = torch.empty(tiles * stride, device=self.runtime.device)

    def _check_tokens(self, t: torch.Tensor, what: str) -> int:
        if (t.dim() != 2 or t.shape[1] != self.d_model or t.dtype != torch.float32 or t.device != self.runtime._y.device
                or not t.is_contiguous()):
            raise ValueError(f"expected a contiguous float32 [N, d_model] tensor {what} on the runtime's device")
        if not 1 <= t.shape[0] <= MAX_TOKENS:
            raise ValueError("unsupported token count")
        return t.shape[0]

    def modes(self, n: int) -> tuple[str, str]:
        """The gather kernels of a forward with z: the runtime's forced modes, else its gather policy (the MFMA path keeps
        no fp32 activations)."""
        runtime = self.runtime
        if runtime.forced_up == "mfma":
            raise ValueError("the training forward runs the gather kernels: force edges or rows")
        up = runtime.forced_up or up_mode(n, self.d_model)
        if up == "edges" and not edges_supported(self.d_model, n):
            up = "rows"
        return up, runtime.forced_down or down_mode(n, self.d_ff)

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.runtime.device).cuda_stream

    # -- the step and its pieces -----------------------------------------------------------------------------------
    def forward(self, index: int, x: torch.Tensor, z: torch.Tensor | None = None) -> torch.Tensor:
        """y[N, d_model] of layer ``index`` (a view of the runtime's output buffer).

        Without ``z``: the inference runtime's own call, unchanged. With ``z`` (contiguous float32 on the device, at least
        d_ff * leading_dim(N) entries): the gather forward that also writes ``z`` hidden-major ``[d_ff, leading_dim(N)]``
        and keeps the state the backward needs (``z`` must stay alive until then)."""
        runtime = self.runtime
        if z is None:
            return runtime.forward(index, x)
        n = self._check_tokens(x, "x")
        ld = leading_dim(n)
        if z.dtype != torch.float32 or z.device != runtime._y.device or not z.is_contiguous() or z.numel() < self.d_ff * ld:
            raise ValueError("z must be a contiguous float32 device tensor of at least d_ff * leading_dim(N) entries")
        self.reserve(n)
        up, down = self.modes(n)
        value_type, *model = runtime._args[index]
        x_t, act, y_t, y = runtime._work
        _lib.check(self._lib.hffn_forward_z(_lib.UP_MODES[up], _lib.DOWN_MODES[down], x.data_ptr(), *model, x_t, act, y_t, y,
                                            z.data_ptr(), self.d_model, self.d_ff, *runtime._nnz[index], n, ld, self._stream()),
                   f"forward with z ({up}, {down})")
        self.calls[up, down] += 1
        self._saved = (index, n, z.data_ptr(), sum(runtime.calls.values()))
        return runtime._y[:n]

    def backward(self, index: int, gy: torch.Tensor) -> torch.Tensor:
        """Compact gradients of layer ``index`` (see ``gradients``) and gx[N, d_model] (a view of the step's buffer) for
        the upstream gradient gy[N, d_model] of the last forward with a z buffer."""
        runtime = self.runtime
        if self._saved is None or self._saved[0] != index or self._saved[3] != sum(runtime.calls.values()):
            raise RuntimeError("backward must follow a forward of the same layer with a z buffer, with no forward in between")
        _, n, z_ptr, _ = self._saved
        if self._check_tokens(gy, "gy") != n:
            raise ValueError("gy must have the N of the forward")
        lib, stream, ld = self._lib, self._stream(), leading_dim(n)
        params, supports, grads = runtime._tensors[index], self._supports[index], self._grads[index]
        values = self._transposed_values[index]
        x_t, act, _, _ = runtime._work
        d, h = self.d_model, self.d_ff
        _lib.check(lib.hffn_transpose(gy.data_ptr(), self._gy_t.data_ptr(), n, d, d, ld, stream), "gy transpose")
        _lib.check(lib.hffn_gather_values(params["out_val"].data_ptr(), supports["hid_pos"].data_ptr(), values["hid_val"].data_ptr(),
                                          values["hid_val"].numel(), stream), "down values, hidden-major")
        _lib.check(lib.hffn_gather_values(params["up_val"].data_ptr(), supports["in_pos"].data_ptr(), values["in_val"].data_ptr(),
                                          values["in_val"].numel(), stream), "up values, input-major")
        dense = self.grad_mode(n) == "dense"
        if dense:
            self._reserve_dense(n)  # a forced mode may need it first
        tiles = 1 if dense else grad_tiles(n)
        if tiles == 1:   # the tile partial is the gradient (and the dense products write the gradients themselves)
            stride = 0
            g_down, gb_down, g_up, gb_up = (grads[name].data_ptr() for name in ("out_val", "b_down", "up_val", "b_up"))
        else:
            c1, c2, c3, stride = self._columns[index]
            ws = self._partials.data_ptr()
            g_down, gb_down, g_up, gb_up = ws, ws + 4 * c1, ws + 4 * c2, ws + 4 * c3
        if dense:
            work, work_bytes = self._dense_work.data_ptr(), self._dense_work.numel()
            _lib.check(lib.hffn_grad_dense(self._gy_t.data_ptr(), act, params["out_offsets"].data_ptr(), params["out_hidden"].data_ptr(),
                                           g_down, gb_down, d, h, n, ld, work, work_bytes, stream), "grad_down (dense)")
        else:
            _lib.check(lib.hffn_grad_sddmm(self._gy_t.data_ptr(), act, params["out_offsets"].data_ptr(), params["out_hidden"].data_ptr(),
                                           g_down, gb_down, d, n, ld, stride, stream), "grad_down")
        _lib.check(lib.hffn_grad_hidden(gy.data_ptr(), self._gy_t.data_ptr(), z_ptr, supports["hid_offsets"].data_ptr(),
                                        supports["hid_output"].data_ptr(), values["hid_val"].data_ptr(), self._gz.data_ptr(),
                                        d, h, values["hid_val"].numel(), n, ld, stream), "grad_hidden")
        if dense:
            _lib.check(lib.hffn_grad_dense(self._gz.data_ptr(), x_t, params["up_offsets"].data_ptr(), params["up_idx"].data_ptr(),
                                           g_up, gb_up, h, d, n, ld, work, work_bytes, stream), "grad_up (dense)")
        else:
            _lib.check(lib.hffn_grad_sddmm(self._gz.data_ptr(), x_t, params["up_offsets"].data_ptr(), params["up_idx"].data_ptr(),
                                           g_up, gb_up, h, n, ld, stride, stream), "grad_up")
        if tiles > 1:
            c1, c2, c3, stride = self._columns[index]
            _lib.check(lib.hffn_reduce_tiles(self._partials.data_ptr(), stride, tiles, c1, c2, c3, grads["out_val"].data_ptr(),
                                             grads["b_down"].data_ptr(), grads["up_val"].data_ptr(), grads["b_up"].data_ptr(),
                                             stream), "reduce_tiles")
        _lib.check(lib.hffn_grad_x(self._gz.data_ptr(), supports["in_offsets"].data_ptr(), supports["in_hidden"].data_ptr(),
                                   values["in_val"].data_ptr(), self._gx_t.data_ptr(), self._gx.data_ptr(), d, h,
                                   values["in_val"].numel(), n, ld, stream),
                   "grad_x")
        return self._gx[:n]

    def adamw(self, index: int) -> None:
        """One AdamW update of the four compact arrays of layer ``index`` from the gradients of the last backward."""
        self.steps[index] += 1
        k = self.steps[index]
        beta1, beta2 = self.betas
        scalars = (self.lr * self.weight_decay, beta1, 1.0 - beta1, beta2, 1.0 - beta2, self.lr / (1.0 - beta1 ** k),
                   math.sqrt(1.0 - beta2 ** k), self.eps)   # float64 on the host, float32 on the device
        params, grads, moments = self.runtime._tensors[index], self._grads[index], self._moments[index]
        stream = self._stream()
        for name in PARAMETERS:
            p = params[name]
            m, v = moments[name]
            _lib.check(self._lib.hffn_adamw(p.data_ptr(), grads[name].data_ptr(), m.data_ptr(), v.data_ptr(), p.numel(), *scalars,
                                            stream), f"adamw {name}")
        self.runtime.invalidate_planes(index)

    def step(self, index: int, x: torch.Tensor, gy: torch.Tensor) -> torch.Tensor:
        """Forward (z in the step's buffer), backward, AdamW. Returns gx (a view of the step's buffer). A larger N than
        reserved grows the buffers first (counted in ``growths``)."""
        self.reserve(self._check_tokens(x, "x"))
        self.forward(index, x, self._z)
        gx = self.backward(index, gy)
        self.adamw(index)
        return gx

    # -- read access (views, no copy) ------------------------------------------------------------------------------
    def parameters(self, index: int) -> dict[str, torch.Tensor]:
        return {name: self.runtime._tensors[index][name] for name in PARAMETERS}

    def gradients(self, index: int) -> dict[str, torch.Tensor]:
        """Keyed by parameter: ``up_val`` hidden-major slot order, ``out_val`` output-major edge order, as the runtime."""
        return self._grads[index]

    def moments(self, index: int) -> dict[str, tuple[torch.Tensor, torch.Tensor]]:
        return self._moments[index]

    def supports(self, index: int) -> dict[str, torch.Tensor]:
        return self._supports[index]

    def activations(self, n: int) -> dict[str, torch.Tensor]:
        """z, h, gz hidden-major [d_ff, N] (strided views of the [d_ff, leading_dim(N)] buffers) and gx [N, d_model] of
        the last step on N tokens."""
        ld = leading_dim(n)
        def hidden(buffer):
            return buffer[:self.d_ff * ld].view(self.d_ff, ld)[:, :n]
        return {"z": hidden(self._z), "h": hidden(self.runtime._act), "gz": hidden(self._gz), "gx": self._gx[:n]}

    def nbytes(self, index: int) -> dict[str, int]:
        """Bytes of layer ``index``: values, gradients, moments, indices (runtime and transposed supports, with the values
        in the transposed orders); dense workspace (with the dense sampled products' planes and partials); the tile
        partials (shared, allocated size)."""
        def size(tensors) -> int:
            return sum(t.numel() * t.element_size() for t in tensors)
        params = self.runtime._tensors[index]
        return {"values": size(params[name] for name in PARAMETERS),
                "gradients": size(self._grads[index].values()),
                "moments": size(t for pair in self._moments[index].values() for t in pair),
                "indices": size(params[name] for name in ("up_offsets", "up_idx", "out_offsets", "out_hidden"))
                + size(self._supports[index].values()) + size(self._transposed_values[index].values()),
                "workspace": self.runtime.workspace_bytes() + size((self._z, self._gz, self._gy_t, self._gx_t, self._gx))
                + self._dense_bytes,
                "partials": size((self._partials,)) if self._partials is not None else 0}
