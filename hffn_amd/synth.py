"""Seeded synthetic HFFN layers in the canonical hidden-major compact layout, and their inputs.

Two families:

* the three fingerprinted test layers of the reference (``CASES``), regenerated with numpy's PCG64
  stream in exactly the order the reference draws it, so that the SHA-256 pinned by the reference
  (``runtime/common/ffn/reference/fingerprints.json:4-6``) identifies them
  (procedure: ``runtime/common/ffn/hffn_ffn_layers/synth.py:53-86``, inputs ``:83-86``);
* the workload layers (``WORKLOADS``): the isolated-layer shapes that the benchmarks and the
  parity tests run (Pythia-70M/410M/1.4B/2.8B shapes at 20-80 % density), drawn with a
  vectorised generator of this package (top-k of uniform keys per neuron for uniform supports,
  Gumbel/Efraimidis-Spirakis keys for the Zipf-biased ones), pinned by the digests in
  ``tests/golden``.

Nothing is stored: every array is regenerated from ``(case, seed)``. Layers hold float32 values;
a ``bf16`` layer holds float32 values that are exactly representable in bfloat16 (round to
nearest even), so the float64 oracle and the device store see the same numbers.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field

import numpy as np

N_GROUPS = 4


@dataclass(frozen=True)
class Case:
    """A reference test layer: ``runtime/common/ffn/hffn_ffn_layers/synth.py:15-35``."""
    name: str
    d_model: int
    d_ff: int
    up_degree: int
    down_degree: int
    irregular: bool
    seed: int


CASES = {
    case.name: case
    for case in (
        Case("homog_256_1024", 256, 1024, 26, 26, False, 1001),
        Case("homog_512_2048", 512, 2048, 51, 51, False, 1002),
        Case("irreg_512_2048", 512, 2048, 51, 51, True, 1003),
    )
}


@dataclass(frozen=True)
class CompactLayer:
    """Hidden-major compact FFN: neuron ``r`` owns up slots and down slots ``[offsets[r], offsets[r+1])``.

    Field names, order and dtypes follow ``runtime/common/ffn/hffn_ffn_layers/synth.py:38-50``; ``value_dtype``
    (``"float32"`` or ``"bf16"``) is the storage type of ``up_val``/``down_val`` on the device."""
    d_model: int
    d_ff: int
    groups: np.ndarray        # int32[5]
    up_offsets: np.ndarray    # int32[d_ff + 1]
    up_idx: np.ndarray        # int16[nnz_up]
    up_val: np.ndarray        # float32[nnz_up]
    b_up: np.ndarray          # float32[d_ff]
    down_offsets: np.ndarray  # int32[d_ff + 1]
    down_idx: np.ndarray      # int16[nnz_down]
    down_val: np.ndarray      # float32[nnz_down]
    b_down: np.ndarray        # float32[d_model]
    value_dtype: str = field(default="float32")


# ----------------------------------------------------------------------------- reference test layers

def _case_degrees(rng: np.random.Generator, case: Case, degree: int) -> np.ndarray:
    if not case.irregular:
        return np.full(case.d_ff, degree, dtype=np.int64)
    return rng.integers(0, min(2 * degree, case.d_model) + 1, size=case.d_ff, dtype=np.int64)


def _case_side(rng: np.random.Generator, degrees: np.ndarray, d_model: int, scale: float):
    offsets = np.zeros(degrees.size + 1, dtype=np.int32)
    np.cumsum(degrees, out=offsets[1:])
    idx = np.empty(int(offsets[-1]), dtype=np.int16)
    for r, k in enumerate(degrees.tolist()):
        idx[offsets[r]:offsets[r + 1]] = np.sort(rng.choice(d_model, size=k, replace=False))
    val = (rng.standard_normal(idx.size) * scale).astype(np.float32)
    return offsets, idx, val


def _groups(d_ff: int) -> np.ndarray:
    return np.array([(g * d_ff) // N_GROUPS for g in range(N_GROUPS + 1)], dtype=np.int32)


def make_layer(case: Case) -> CompactLayer:
    """The test layer of ``case``; draw order as ``runtime/common/ffn/hffn_ffn_layers/synth.py:71-80``."""
    rng = np.random.default_rng(case.seed)
    up_deg = _case_degrees(rng, case, case.up_degree)
    down_deg = _case_degrees(rng, case, case.down_degree)
    up = _case_side(rng, up_deg, case.d_model, 1.0 / np.sqrt(case.up_degree))
    down = _case_side(rng, down_deg, case.d_model, 1.0 / np.sqrt(case.down_degree))
    b_up = (rng.standard_normal(case.d_ff) * 0.1).astype(np.float32)
    b_down = (rng.standard_normal(case.d_model) * 0.1).astype(np.float32)
    return CompactLayer(case.d_model, case.d_ff, _groups(case.d_ff), up[0], up[1], up[2], b_up, down[0], down[1], down[2], b_down)


def make_input(case, n: int) -> np.ndarray:
    """Token-major float32 input ``[n, d_model]`` from PCG64 seeded ``[seed, n]``
    (``runtime/common/ffn/hffn_ffn_layers/synth.py:83-86``); ``case`` is a ``Case`` or a ``Workload``."""
    rng = np.random.default_rng([case.seed, n])
    return np.ascontiguousarray(rng.standard_normal((n, case.d_model)).astype(np.float32))


FIELDS = ("groups", "up_offsets", "up_idx", "up_val", "b_up", "down_offsets", "down_idx", "down_val", "b_down")
FINGERPRINT_N = (1, 2, 4, 7, 8, 16, 32, 64, 96, 128)


def fingerprint(layer: CompactLayer, case, inputs: tuple[int, ...] = FINGERPRINT_N) -> str:
    """SHA-256 of the layer arrays (``FIELDS`` order) then of ``make_input(case, n)`` for each ``n``
    (``runtime/common/ffn/hffn_ffn_layers/layers.py:21-44``)."""
    digest = hashlib.sha256()
    for name in FIELDS:
        digest.update(np.ascontiguousarray(getattr(layer, name)).tobytes())
    for n in inputs:
        digest.update(make_input(case, n).tobytes())
    return digest.hexdigest()


# ----------------------------------------------------------------------------- workload layers

@dataclass(frozen=True)
class Workload:
    """An isolated-layer workload. ``degree`` is the support size of every neuron (uniform supports), or
    the mean of a clipped normal when ``degree_std`` is set; ``zipf`` biases the drawn indices towards a
    random subset of inputs (weight ``(rank + 1) ** -zipf`` over a random permutation)."""
    name: str
    d_model: int
    d_ff: int
    degree: int
    seed: int
    w_std: float = 0.02
    b_up_std: float = 0.0
    b_down_std: float = 0.0
    value_dtype: str = "float32"
    degree_std: float = 0.0
    degree_min: int = 0
    zipf: float = 0.0
    tokens: tuple[int, ...] = (1,)


WORKLOADS = {
    w.name: w
    for w in (
        Workload("pythia70m_d20", 512, 2048, 102, 101, tokens=(128,)),
        Workload("pythia410m_d50", 1024, 4096, 512, 102, b_up_std=0.01, b_down_std=0.01,
                 tokens=(2048, 1, 4, 8, 16, 32)),
        Workload("pythia1p4b_d20_bf16", 2048, 8192, 410, 103, value_dtype="bf16", tokens=(1, 4, 16)),
        Workload("pythia2p8b_d80_zipf_bf16", 2560, 10240, 2048, 105, value_dtype="bf16",
                 degree_std=300.0, degree_min=256, zipf=1.1, tokens=(4096,)),
    )
}


def round_bf16(values: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16 (ties to even), returned as float32."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    return rounded.astype(np.uint32).view(np.float32)


def _topk_rows(keys: np.ndarray, degrees: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per row, the columns of its ``degrees[row]`` largest keys, ascending; returns (offsets, idx)."""
    rows, cols = keys.shape
    offsets = np.zeros(rows + 1, dtype=np.int32)
    np.cumsum(degrees, out=offsets[1:])
    order = np.argsort(-keys, axis=1, kind="stable")
    mask = np.arange(cols)[None, :] < degrees[:, None]
    chosen = np.where(mask, order, cols)
    chosen.sort(axis=1)
    idx = chosen[chosen < cols].astype(np.int16)
    assert idx.size == offsets[-1]
    return offsets, idx


def _workload_side(rng: np.random.Generator, w: Workload, chunk: int = 2048):
    if w.degree_std:
        degrees = np.clip(np.rint(rng.normal(w.degree, w.degree_std, w.d_ff)), w.degree_min, w.d_model).astype(np.int64)
    else:
        degrees = np.full(w.d_ff, w.degree, dtype=np.int64)
    if w.zipf:
        permutation = rng.permutation(w.d_model)
        weight = np.empty(w.d_model)
        weight[permutation] = (np.arange(w.d_model) + 1.0) ** -w.zipf
        log_weight = np.log(weight / weight.sum())
    offsets_parts, idx_parts = [], []
    for start in range(0, w.d_ff, chunk):
        rows = min(chunk, w.d_ff - start)
        u = rng.random((rows, w.d_model))
        if w.zipf:
            # Gumbel-top-k: weighted sampling without replacement with probabilities proportional to `weight`.
            keys = log_weight[None, :] - np.log(-np.log(np.maximum(u, 1e-300)))
        else:
            keys = u
        offsets, idx = _topk_rows(keys, degrees[start:start + rows])
        offsets_parts.append(offsets)
        idx_parts.append(idx)
    offsets = np.zeros(w.d_ff + 1, dtype=np.int32)
    np.cumsum(degrees, out=offsets[1:])
    idx = np.concatenate(idx_parts)
    val = (rng.standard_normal(idx.size) * w.w_std).astype(np.float32)
    if w.value_dtype == "bf16":
        val = round_bf16(val)
    return offsets, idx, val


def make_workload_layer(w: Workload | str, seed: int | None = None) -> CompactLayer:
    """The layer of a workload (``seed`` overrides the workload's, e.g. for distinct copies of one shape)."""
    if isinstance(w, str):
        w = WORKLOADS[w]
    rng = np.random.default_rng(w.seed if seed is None else seed)
    up = _workload_side(rng, w)
    down = _workload_side(rng, w)
    b_up = (rng.standard_normal(w.d_ff) * w.b_up_std).astype(np.float32)
    b_down = (rng.standard_normal(w.d_model) * w.b_down_std).astype(np.float32)
    return CompactLayer(w.d_model, w.d_ff, _groups(w.d_ff), up[0], up[1], up[2], b_up,
                        down[0], down[1], down[2], b_down, w.value_dtype)


def make_workload_input(w: Workload | str, n: int) -> np.ndarray:
    if isinstance(w, str):
        w = WORKLOADS[w]
    return make_input(w, n)


def layer_digest(layer: CompactLayer) -> str:
    """SHA-256 of the layer arrays only (the workload layers' pin)."""
    digest = hashlib.sha256()
    for name in FIELDS:
        digest.update(np.ascontiguousarray(getattr(layer, name)).tobytes())
    return digest.hexdigest()
