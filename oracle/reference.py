"""float64 oracle of the HFFN forward (test infrastructure; see ``oracle/__init__.py``).

``layer`` is any object with the compact hidden-major fields of ``runtime/common/ffn/hffn_ffn_layers/synth.py:38-50``
(``d_model``, ``d_ff``, ``up_offsets``, ``up_idx``, ``up_val``, ``b_up``, ``down_offsets``, ``down_idx``,
``down_val``, ``b_down``); ``x`` is token-major ``[N, d_model]``. Every function returns ``y[N, d_model]`` in float64.

Three independent formulations:

* ``forward_slots`` - the reference oracle's algorithm (``reference.py:21-38``): z = b_up, then every up slot adds
  ``x[:, idx] * w`` to its owner's row; exact GELU; y = b_down, then every down slot adds ``h[:, owner] * v`` to its
  output's row (``np.add.at``).
* ``forward_dense`` - the closed form of ``runtime/common/pythia/hffn_pythia/oracle.py:17-31``: materialise
  ``W_up[d_ff, d_model]`` and ``W_down[d_model, d_ff]`` (zeros outside the support), ``W_down gelu(W_up x + b_up) +
  b_down`` with BLAS float64 products; used for the large shapes.
* ``forward_loops`` - plain Python loops over tokens, neurons and slots with ``math.erf``, for tiny cases.
"""
from __future__ import annotations

import math

import numpy as np
from scipy.special import erf as _scipy_erf

_math_erf = np.vectorize(math.erf, otypes=[np.float64])

SQRT_HALF = 0.7071067811865476


def gelu_exact(z: np.ndarray) -> np.ndarray:
    """``0.5 z (1 + erf(z / sqrt 2))`` with Python's ``math.erf`` (``reference.py:17-18``)."""
    return 0.5 * z * (1.0 + _math_erf(z * SQRT_HALF))


def gelu_fast(z: np.ndarray) -> np.ndarray:
    """The same GELU with ``scipy.special.erf`` (vectorised; agrees with ``math.erf`` to a few float64 ulps)."""
    return 0.5 * z * (1.0 + _scipy_erf(z * SQRT_HALF))


def owners(offsets: np.ndarray, d_ff: int) -> np.ndarray:
    """Hidden neuron of each slot: neuron r repeated ``offsets[r+1] - offsets[r]`` times."""
    return np.repeat(np.arange(d_ff), np.diff(offsets.astype(np.int64)))


def values64(values: np.ndarray) -> np.ndarray:
    return np.asarray(values, dtype=np.float32).astype(np.float64)


def forward_slots(layer, x_nt: np.ndarray, gelu=gelu_exact) -> np.ndarray:
    x = np.asarray(x_nt, dtype=np.float32).astype(np.float64)
    n = x.shape[0]
    z = np.tile(values64(layer.b_up), (n, 1))
    up_owner = owners(layer.up_offsets, layer.d_ff)
    np.add.at(z.T, up_owner, (x[:, layer.up_idx.astype(np.int64)] * values64(layer.up_val)).T)
    h = gelu(z)
    y = np.tile(values64(layer.b_down), (n, 1))
    down_owner = owners(layer.down_offsets, layer.d_ff)
    np.add.at(y.T, layer.down_idx.astype(np.int64), (h[:, down_owner] * values64(layer.down_val)).T)
    return y


def dense_weights(layer) -> tuple[np.ndarray, np.ndarray]:
    """float64 ``W_up[d_ff, d_model]`` and ``W_down[d_model, d_ff]``, zero outside the support."""
    w_up = np.zeros((layer.d_ff, layer.d_model))
    w_up[owners(layer.up_offsets, layer.d_ff), layer.up_idx.astype(np.int64)] = values64(layer.up_val)
    w_down = np.zeros((layer.d_model, layer.d_ff))
    w_down[layer.down_idx.astype(np.int64), owners(layer.down_offsets, layer.d_ff)] = values64(layer.down_val)
    return w_up, w_down


def forward_dense(layer, x_nt: np.ndarray, weights=None, gelu=gelu_fast) -> np.ndarray:
    w_up, w_down = dense_weights(layer) if weights is None else weights
    x = np.asarray(x_nt, dtype=np.float32).astype(np.float64)
    z = x @ w_up.T + values64(layer.b_up)
    return gelu(z) @ w_down.T + values64(layer.b_down)


def forward_loops(layer, x_nt: np.ndarray) -> np.ndarray:
    """Token by token, neuron by neuron, slot by slot (tiny layers only)."""
    x = np.asarray(x_nt, dtype=np.float32)
    n = x.shape[0]
    up_off, down_off = layer.up_offsets.tolist(), layer.down_offsets.tolist()
    up_idx, down_idx = layer.up_idx.tolist(), layer.down_idx.tolist()
    up_val, down_val = values64(layer.up_val).tolist(), values64(layer.down_val).tolist()
    b_up, b_down = values64(layer.b_up).tolist(), values64(layer.b_down).tolist()
    y = np.zeros((n, layer.d_model))
    for t in range(n):
        row = [float(v) for v in x[t]]
        out = list(b_down)
        for r in range(layer.d_ff):
            z = b_up[r]
            for e in range(up_off[r], up_off[r + 1]):
                z += up_val[e] * row[up_idx[e]]
            a = 0.5 * z * (1.0 + math.erf(z / math.sqrt(2.0)))
            for e in range(down_off[r], down_off[r + 1]):
                out[down_idx[e]] += down_val[e] * a
        y[t] = out
    return y


def forward(layer, x_nt: np.ndarray) -> np.ndarray:
    """The oracle of the tests: the slot walk for small layers, the dense closed form for large ones."""
    if layer.d_model * layer.d_ff * x_nt.shape[0] <= (1 << 26):
        return forward_slots(layer, x_nt, gelu=gelu_fast)
    return forward_dense(layer, x_nt)
