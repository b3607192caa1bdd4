"""float64 oracle of one HFFN training step (test infrastructure; see ``oracle/__init__.py``).

Restates the oracle of ``runtime/gpu/nvidia/ffn/training/train_step.py:56-82`` (forward and backward of the
fixed-support FFN on its compact hidden-major store) and its AdamW closed form (``train_step.py:85-92``):

    z = W_up x + b_up,  h = gelu(z),  y = W_down h + b_down,           (exact-erf GELU)
    gb_down = sum_t gy,  g_down[q] = sum_t gy[t, o_q] h[t, r_q],
    gz = (gy W_down) * gelu'(z),   gelu'(z) = Phi(z) + z phi(z),
    gb_up = sum_t gz,    g_up[e] = sum_t gz[t, r_e] x[t, i_e],
    gx = gz W_up.

Here the weights are scipy sparse matrices of the compact stores (duplicate slots summed, as the slot walk sums them)
and the sampled gradients are entries of the dense float64 products ``gy^T h`` and ``gz^T x``; every group comes back
in hidden-major slot order (``g_down`` in the slot order of ``down_idx``). Pinned in ``tests/test_train_oracle.py``
against ``torch.autograd`` in float64 and ``torch.optim.AdamW`` in float64.
"""
from __future__ import annotations

import math

import numpy as np
import scipy.sparse as sp
from scipy.special import erf

from .reference import owners, values64

SQRT_HALF = 0.7071067811865476
INV_SQRT_2PI = 0.3989422804014327


def gelu(z: np.ndarray) -> np.ndarray:
    return 0.5 * z * (1.0 + erf(z * SQRT_HALF))


def gelu_grad(z: np.ndarray) -> np.ndarray:
    """0.5 (1 + erf(z / sqrt 2)) + z exp(-z^2 / 2) / sqrt(2 pi) (``train_step.py:52-53``)."""
    return 0.5 * (1.0 + erf(z * SQRT_HALF)) + z * np.exp(-0.5 * z * z) * INV_SQRT_2PI


def _params(layer, params: dict | None) -> dict:
    if params is not None:
        return {name: np.asarray(value, dtype=np.float64) for name, value in params.items()}
    return {"up_val": values64(layer.up_val), "b_up": values64(layer.b_up), "down_val": values64(layer.down_val),
            "b_down": values64(layer.b_down)}


def step_groups(layer, x: np.ndarray, gy: np.ndarray, params: dict | None = None) -> dict[str, np.ndarray]:
    """Every group of one step for x, gy token-major [N, d_model]: ``y`` [N, d], ``gz`` [d_ff, N], ``gx`` [N, d],
    ``g_up``, ``gb_up``, ``g_down`` (hidden-major slot order), ``gb_down``. ``params`` (hidden-major float64 ``up_val``,
    ``b_up``, ``down_val``, ``b_down``) overrides the layer's values."""
    p = _params(layer, params)
    d, h = layer.d_model, layer.d_ff
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    gy = np.asarray(gy, dtype=np.float32).astype(np.float64)
    up_owner, up_input = owners(layer.up_offsets, h), layer.up_idx.astype(np.int64)
    down_owner, down_output = owners(layer.down_offsets, h), layer.down_idx.astype(np.int64)
    w_up = sp.csr_matrix((p["up_val"], (up_owner, up_input)), shape=(h, d))          # duplicates summed
    w_down = sp.csr_matrix((p["down_val"], (down_output, down_owner)), shape=(d, h))
    z = np.asarray((w_up @ x.T).T) + p["b_up"]                                         # [N, d_ff]
    act = gelu(z)
    y = np.asarray((w_down @ act.T).T) + p["b_down"]
    g_down_dense = gy.T @ act                                                           # [d, d_ff]
    gz = np.asarray((w_down.T @ gy.T).T) * gelu_grad(z)                                 # [N, d_ff]
    g_up_dense = gz.T @ x                                                               # [d_ff, d]
    gx = np.asarray((w_up.T @ gz.T).T)
    return {"y": y, "gz": gz.T.copy(), "gx": gx, "g_up": g_up_dense[up_owner, up_input], "gb_up": gz.sum(0),
            "g_down": g_down_dense[down_output, down_owner], "gb_down": gy.sum(0)}


def adamw_closed_form(p, g, m, v, step: int, lr: float, betas: tuple[float, float], eps: float, weight_decay: float):
    """One AdamW update in float64 (decoupled decay, bias correction; ``train_step.py:85-92``): returns (p, m, v)."""
    b1, b2 = betas
    m = b1 * m + (1.0 - b1) * g
    v = b2 * v + (1.0 - b2) * g * g
    p = p * (1.0 - lr * weight_decay) - lr * (m / (1.0 - b1 ** step)) / (np.sqrt(v / (1.0 - b2 ** step)) + eps)
    return p, m, v


def output_major_order(layer) -> np.ndarray:
    """Output-major edge position -> hidden-major down slot (the stable argsort of ``down_idx``)."""
    return np.argsort(layer.down_idx.astype(np.int64), kind="stable")


def step_groups_loops(layer, x: np.ndarray, gy: np.ndarray) -> dict[str, np.ndarray]:
    """The same groups by plain Python loops over tokens and slots with ``math.erf`` (tiny cases only)."""
    d, h = layer.d_model, layer.d_ff
    up_owner, down_owner = owners(layer.up_offsets, h), owners(layer.down_offsets, h)
    w, b, v, c = (values64(a) for a in (layer.up_val, layer.b_up, layer.down_val, layer.b_down))
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    gy = np.asarray(gy, dtype=np.float32).astype(np.float64)
    n = x.shape[0]
    out = {"y": np.zeros((n, d)), "gz": np.zeros((h, n)), "gx": np.zeros((n, d)), "g_up": np.zeros(len(w)),
           "gb_up": np.zeros(h), "g_down": np.zeros(len(v)), "gb_down": np.zeros(d)}
    for t in range(n):
        z = [float(b[r]) for r in range(h)]
        for e in range(len(w)):
            z[up_owner[e]] += w[e] * x[t, layer.up_idx[e]]
        act = [0.5 * zr * (1.0 + math.erf(zr * SQRT_HALF)) for zr in z]
        for o in range(d):
            out["y"][t, o] = c[o]
            out["gb_down"][o] += gy[t, o]
        dh = [0.0] * h
        for q in range(len(v)):
            o, r = int(layer.down_idx[q]), down_owner[q]
            out["y"][t, o] += v[q] * act[r]
            out["g_down"][q] += gy[t, o] * act[r]
            dh[r] += v[q] * gy[t, o]
        for r in range(h):
            zr = z[r]
            grad = dh[r] * (0.5 * (1.0 + math.erf(zr * SQRT_HALF)) + zr * math.exp(-0.5 * zr * zr) * INV_SQRT_2PI)
            out["gz"][r, t] = grad
            out["gb_up"][r] += grad
        for e in range(len(w)):
            r, i = up_owner[e], int(layer.up_idx[e])
            out["g_up"][e] += out["gz"][r, t] * x[t, i]
            out["gx"][t, i] += w[e] * out["gz"][r, t]
    return out
