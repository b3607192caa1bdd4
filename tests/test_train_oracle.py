"""The float64 training oracle (``oracle.train``) pinned on the CPU, and the host logic of the training runtime.

* every group of one step against ``torch.autograd`` in float64 on the dense weights (an independent derivation of the
  backward), on a random layer and on the reference test layer ``homog_256_1024``;
* the sparse closed form against plain Python loops on a tiny layer with repeated indices in a row;
* the AdamW closed form against ``torch.optim.AdamW`` in float64 over several steps;
* planted mistakes in the oracle (GELU derivative without its density term, a dropped bias gradient, a transposed
  sampled product) are caught by the autograd comparison;
* the token tiles of the gather sampled products.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hffn_amd import synth
from hffn_amd.train_runtime import grad_tiles
from oracle import train as oracle_train
from oracle.reference import owners

HYPER = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2)


def _random_layer(d: int, h: int, per_row: int, seed: int, repeats: bool = False) -> synth.CompactLayer:
    rng = np.random.default_rng(seed)
    offsets = np.arange(h + 1, dtype=np.int32) * per_row
    if repeats:
        up_idx = rng.integers(0, d, h * per_row).astype(np.int16)
        down_idx = rng.integers(0, d, h * per_row).astype(np.int16)
    else:
        up_idx = np.concatenate([np.sort(rng.choice(d, per_row, replace=False)) for _ in range(h)]).astype(np.int16)
        down_idx = np.concatenate([np.sort(rng.choice(d, per_row, replace=False)) for _ in range(h)]).astype(np.int16)
    f = lambda size, s: (rng.standard_normal(size) * s).astype(np.float32)  # noqa: E731
    return synth.CompactLayer(d, h, synth._groups(h), offsets, up_idx, f(h * per_row, 0.3), f(h, 0.1), offsets, down_idx,
                              f(h * per_row, 0.3), f(d, 0.1))


def _autograd_groups(layer, x: np.ndarray, gy: np.ndarray) -> dict:
    """One step by torch.autograd in float64 on the dense weights (zeros outside the support)."""
    f64 = torch.float64
    up_owner, down_owner = owners(layer.up_offsets, layer.d_ff), owners(layer.down_offsets, layer.d_ff)
    w_up = torch.zeros(layer.d_ff, layer.d_model, dtype=f64)
    w_up[up_owner, layer.up_idx.astype(np.int64)] = torch.from_numpy(layer.up_val.astype(np.float64))
    w_down = torch.zeros(layer.d_model, layer.d_ff, dtype=f64)
    w_down[layer.down_idx.astype(np.int64), down_owner] = torch.from_numpy(layer.down_val.astype(np.float64))
    w_up.requires_grad_()
    w_down.requires_grad_()
    b_up = torch.from_numpy(layer.b_up.astype(np.float64)).requires_grad_()
    b_down = torch.from_numpy(layer.b_down.astype(np.float64)).requires_grad_()
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_()
    z = xt @ w_up.T + b_up
    z.retain_grad()
    y = torch.nn.functional.gelu(z, approximate="none") @ w_down.T + b_down
    y.backward(torch.from_numpy(gy.astype(np.float64)))
    return {"y": y.detach().numpy(), "gz": z.grad.T.numpy(), "gx": xt.grad.numpy(),
            "g_up": w_up.grad[up_owner, layer.up_idx.astype(np.int64)].numpy(), "gb_up": b_up.grad.numpy(),
            "g_down": w_down.grad[layer.down_idx.astype(np.int64), down_owner].numpy(), "gb_down": b_down.grad.numpy()}


def _inputs(layer, n: int, seed: int):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, layer.d_model)).astype(np.float32),
            (0.1 * rng.standard_normal((n, layer.d_model))).astype(np.float32))


def _assert_groups_close(got: dict, expected: dict, rtol: float = 1e-10) -> None:
    for name, value in expected.items():
        scale = max(1.0, float(np.abs(value).max()))
        assert float(np.abs(got[name] - value).max()) <= rtol * scale, name


@pytest.mark.parametrize("n", [1, 7, 64])
def test_oracle_matches_autograd_random_layer(n):
    layer = _random_layer(48, 96, 12, seed=n)
    x, gy = _inputs(layer, n, seed=100 + n)
    _assert_groups_close(oracle_train.step_groups(layer, x, gy), _autograd_groups(layer, x, gy))


def test_oracle_matches_autograd_reference_layer():
    layer = synth.make_layer(synth.CASES["homog_256_1024"])
    x, gy = _inputs(layer, 33, seed=5)
    _assert_groups_close(oracle_train.step_groups(layer, x, gy), _autograd_groups(layer, x, gy))


def test_oracle_matches_loops_with_repeated_indices():
    layer = _random_layer(6, 5, 4, seed=3, repeats=True)
    assert any(len(set(layer.up_idx[r * 4:(r + 1) * 4])) < 4 for r in range(5))  # a row repeats an input
    x, gy = _inputs(layer, 3, seed=9)
    _assert_groups_close(oracle_train.step_groups(layer, x, gy), oracle_train.step_groups_loops(layer, x, gy), rtol=1e-12)


def test_adamw_closed_form_matches_torch():
    rng = np.random.default_rng(11)
    p0 = rng.standard_normal(50)
    grads = [rng.standard_normal(50) for _ in range(4)]
    param = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    optimiser = torch.optim.AdamW([param], foreach=False, fused=False, **HYPER)
    p, m, v = p0.copy(), np.zeros(50), np.zeros(50)
    for k, g in enumerate(grads, start=1):
        param.grad = torch.from_numpy(g.copy())
        optimiser.step()
        p, m, v = oracle_train.adamw_closed_form(p, g, m, v, k, **HYPER)
        assert np.allclose(param.detach().numpy(), p, rtol=1e-13, atol=1e-15)
        state = optimiser.state[param]
        assert np.allclose(state["exp_avg"].numpy(), m, rtol=1e-13) and np.allclose(state["exp_avg_sq"].numpy(), v, rtol=1e-13)


@pytest.mark.parametrize("mistake", ["no_density_term", "no_bias_gradient", "transposed_product"])
def test_planted_mistakes_are_caught(mistake, monkeypatch):
    layer = _random_layer(32, 64, 8, seed=21)
    x, gy = _inputs(layer, 9, seed=22)
    expected = _autograd_groups(layer, x, gy)
    if mistake == "no_density_term":
        monkeypatch.setattr(oracle_train, "gelu_grad", lambda z: 0.5 * (1.0 + oracle_train.erf(z * oracle_train.SQRT_HALF)))
        got = oracle_train.step_groups(layer, x, gy)
    else:
        got = dict(oracle_train.step_groups(layer, x, gy))
        if mistake == "no_bias_gradient":
            got["gb_up"] = np.zeros_like(got["gb_up"])
        else:  # g_up sampled at (input, owner) instead of (owner, input)
            gz, xx = got["gz"], x.astype(np.float64)
            dense = gz @ xx                       # [d_ff, d]
            up_owner = owners(layer.up_offsets, layer.d_ff)
            got["g_up"] = dense.T[layer.up_idx.astype(np.int64) % layer.d_model, up_owner % layer.d_model]
    with pytest.raises(AssertionError):
        _assert_groups_close(got, expected)


def test_grad_tiles():
    assert [grad_tiles(n) for n in (1, 255, 256, 257, 512, 2100)] == [1, 1, 1, 2, 2, 9]
