"""The training step on the GPU (``HFFNTrainRuntime``) against the float64 oracle, with the gates of
runtime/gpu/nvidia/ffn/training/check.py:1-12:

1. the forward without z is the inference runtime's call, bit for bit; with z, y is the same gather forward's bits;
2. every group (y, gb_down, g_down, gz, g_up, gb_up, gx) within 10x the float64 distance of the dense float32
   control (PyTorch autograd on the dense masked weights), with a relative floor of 1e-7 (train_step.py:24-27);
3. one AdamW update against its float64 closed form fed the build's own gradient, on the conditioned entries
   (|g| >= 100x the control's group distance), relative 1e-5;
4. the same bits twice from the same state; supports and offsets unchanged;
5. five steps, each update against the closed form from the build's own pre-update state (relative 1e-5);
then: no buffer growth in a step after ``reserve``, the ordering check of ``backward``, and the MFMA path of the
inference runtime reading the updated values.
N covers one tile (1, 33, 100, 128), a one-token last tile (257), partial last tiles (300, 2100) and exact tiles (512).
The sampled products run as gathers (``gather``) or as dense split-fp16 MFMA products sampled at the support
(``dense``, the policy's choice from 64 tokens on the 512 x 2048 layers); cases force either where the policy would
not take it, so both meet every gate. The forward with z, gz and gx run as gathers or on the planes (``mfma``, the
policy's choice from 64 tokens where the streamed GEMM takes N); planes cases check gate 1 against the inference
runtime's MFMA call (the same products: its bits).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from hffn_amd import synth
from hffn_amd.ffn import hip_layer
from hffn_amd.runtime import HFFNRuntime
from hffn_amd.train_runtime import HFFNTrainRuntime
from oracle import train as oracle_train
from oracle.reference import owners

pytestmark = pytest.mark.gpu

HYPER = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2)
GROUPS = ("y", "gb_down", "g_down", "gz", "g_up", "gb_up", "gx")
GATE2_FACTOR, GATE2_FLOOR = 10.0, 1e-7
GATE3_CONDITIONING, GATE3_RELATIVE = 100.0, 1e-5
CASES = ([("homog_256_1024", n, None, None) for n in (1, 33, 100, 128, 257, 300, 512, 2100)]
         + [("homog_256_1024", 2100, None, "gather"), ("irreg_512_2048", 4, None, None), ("irreg_512_2048", 300, None, "gather"),
            ("irreg_512_2048", 300, "gather", "gather"), ("irreg_512_2048", 33, "dense", "gather"), ("irreg_512_2048", 300, None, "mfma"),
            ("irreg_512_2048", 33, None, "mfma"), ("homog_512_2048", 64, None, None), ("homog_512_2048", 2100, None, None),
            ("homog_512_2048", 2100, "gather", "gather")])


def make_gy(case, n: int, salt: int) -> torch.Tensor:
    rng = np.random.Generator(np.random.PCG64([case.seed, n, 7919, salt]))
    return torch.from_numpy(rng.standard_normal((n, case.d_model)).astype(np.float32) * 0.1)


def _dense(layer, device):
    up_owner = torch.from_numpy(owners(layer.up_offsets, layer.d_ff)).to(device)
    down_owner = torch.from_numpy(owners(layer.down_offsets, layer.d_ff)).to(device)
    up_idx = torch.from_numpy(layer.up_idx.astype(np.int64)).to(device)
    down_idx = torch.from_numpy(layer.down_idx.astype(np.int64)).to(device)
    w_up = torch.zeros(layer.d_ff, layer.d_model, device=device)
    w_up[up_owner, up_idx] = torch.from_numpy(layer.up_val).to(device)
    w_down = torch.zeros(layer.d_model, layer.d_ff, device=device)
    w_down[down_idx, down_owner] = torch.from_numpy(layer.down_val).to(device)
    return w_up, w_down, (up_owner, up_idx, down_owner, down_idx)


def control_groups(layer, x, gy) -> dict:
    """The dense float32 step by autograd on the device (train_step.py:128-143): every group, hidden-major slot order."""
    w_up, w_down, (up_owner, up_idx, down_owner, down_idx) = _dense(layer, x.device)
    w_up.requires_grad_()
    w_down.requires_grad_()
    b_up = torch.from_numpy(layer.b_up.copy()).to(x.device).requires_grad_()
    b_down = torch.from_numpy(layer.b_down.copy()).to(x.device).requires_grad_()
    xg = x.detach().clone().requires_grad_()
    z = F.linear(xg, w_up, b_up)
    z.retain_grad()
    y = F.linear(F.gelu(z, approximate="none"), w_down, b_down)
    y.backward(gy)
    out = {"y": y.detach(), "gz": z.grad.T.contiguous(), "gx": xg.grad, "g_up": w_up.grad[up_owner, up_idx],
           "gb_up": b_up.grad, "g_down": w_down.grad[down_idx, down_owner], "gb_down": b_down.grad}
    return {k: v.double().cpu().numpy() for k, v in out.items()}


def build_groups(train, layer, n: int) -> dict:
    """The seven groups of the build's last step, hidden-major slot order (g_down back from output-major)."""
    perm = oracle_train.output_major_order(layer)
    grads, acts = train.gradients(0), train.activations(n)
    g_down = np.empty(perm.size)
    g_down[perm] = grads["out_val"].double().cpu().numpy()
    return {"y": train.runtime._y[:n].double().cpu().numpy(), "gb_down": grads["b_down"].double().cpu().numpy(), "g_down": g_down,
            "gz": acts["gz"].double().cpu().numpy(), "g_up": grads["up_val"].double().cpu().numpy(),
            "gb_up": grads["b_up"].double().cpu().numpy(), "gx": acts["gx"].double().cpu().numpy()}


def hidden_major_state(train, layer) -> dict:
    """(value, m, v) per parameter as float64 numpy, down side mapped back to hidden-major slot order."""
    perm = oracle_train.output_major_order(layer)
    params, moments = train.parameters(0), train.moments(0)
    out = {}
    for name in ("up_val", "b_up", "out_val", "b_down"):
        tensors = [t.double().cpu().numpy() for t in (params[name], *moments[name])]
        if name == "out_val":
            back = []
            for t in tensors:
                b = np.empty_like(t)
                b[perm] = t
                back.append(b)
            tensors = back
        out["down_val" if name == "out_val" else name] = tuple(tensors)
    return out


GRAD_OF = {"up_val": "g_up", "b_up": "gb_up", "down_val": "g_down", "b_down": "gb_down"}


def _update_errors(pre: dict, post: dict, groups: dict, masks: dict, step: int) -> float:
    worst = 0.0
    for p, g in GRAD_OF.items():
        p0, m0, v0 = pre[p]
        ref_p, ref_m, ref_v = oracle_train.adamw_closed_form(p0, groups[g], m0, v0, step, **HYPER)
        got_p, got_m, got_v = post[p]
        mask = masks[g]
        if not mask.any():
            continue
        scale_p = np.maximum(np.maximum(np.abs(ref_p), np.abs(p0)), HYPER["lr"])
        scale_m = np.maximum(np.maximum(np.abs(ref_m), HYPER["betas"][0] * np.abs(m0)), (1 - HYPER["betas"][0]) * np.abs(groups[g]))
        for got, ref, scale in ((got_p, ref_p, scale_p), (got_m, ref_m, scale_m), (got_v, ref_v, np.abs(ref_v))):
            worst = max(worst, float((np.abs(got - ref) / np.maximum(scale, 1e-30))[mask].max()))
    return worst


@pytest.mark.parametrize("name,n,grad,mode", CASES)
def test_training_gates(name, n, grad, mode, device):
    case = synth.CASES[name]
    layer = synth.make_layer(case)
    x = torch.from_numpy(synth.make_input(case, n)).to(device)
    gy = make_gy(case, n, 0).to(device)
    baseline = HFFNRuntime([hip_layer(layer)], device, dense=True)
    train = HFFNTrainRuntime(HFFNRuntime([hip_layer(layer)], device, dense=True), **HYPER, max_tokens=max(n, 2048))
    train.forced_grad = grad
    train.forced_train = mode
    if name.endswith("512_2048") and grad is None:
        assert train.grad_mode(n) == ("dense" if n >= 64 else "gather")
    if name.endswith("512_2048") and mode is None:
        assert train.train_mode(n) == ("mfma" if n >= 64 else "gather")
    planes = train.train_mode(n) == "mfma"
    train.reserve(n)
    # gate 1: the inference call is untouched; the forward with z has the bits of the same gather forward, or on the
    # planes those of the inference MFMA call
    pairs = ((None, None),) if planes else ((None, None), ("edges", "edges"), ("rows", "rows"), ("edges", "rows"), ("rows", "edges"))
    for pair in pairs:
        baseline.force(*pair)
        train.runtime.force(*pair)
        assert torch.equal(baseline.forward(0, x).clone(), train.forward(0, x).clone()), pair
        if pair != (None, None):
            assert torch.equal(train.forward(0, x, train._z).clone(), baseline.forward(0, x)), pair
    if planes:
        baseline.force("mfma", "mfma")
        assert torch.equal(train.forward(0, x, train._z).clone(), baseline.forward(0, x))
        assert train.calls["mfma", "mfma"] == 1
    baseline.force(None, None)
    train.runtime.force(None, None)
    train.reserve(n)
    growths = train.growths
    x_np, gy_np = x.cpu().numpy(), gy.cpu().numpy()
    ref = oracle_train.step_groups(layer, x_np, gy_np)
    control = control_groups(layer, x, gy)
    initial = {k: v.clone() for k, v in train.parameters(0).items()}
    before = hidden_major_state(train, layer)
    train.step(0, x, gy)
    torch.cuda.synchronize()
    assert train.growths == growths, "a step after reserve allocated"
    groups = build_groups(train, layer, n)
    # gate 2
    for g in GROUPS:
        scale = float(np.abs(ref[g]).max())
        d_build, d_control = float(np.abs(groups[g] - ref[g]).max()), float(np.abs(control[g] - ref[g]).max())
        assert d_build <= GATE2_FACTOR * max(d_control, GATE2_FLOOR * scale), (g, d_build, d_control, scale)
    # gate 3
    masks = {g: np.abs(ref[g]) >= GATE3_CONDITIONING * float(np.abs(control[g] - ref[g]).max()) for g in GRAD_OF.values()}
    assert all(mask.any() for mask in masks.values())
    assert _update_errors(before, hidden_major_state(train, layer), groups, masks, 1) <= GATE3_RELATIVE
    # gate 4: the same bits from the same state; supports and offsets unchanged
    first = [t.clone() for t in (train._gx[:n], *train.gradients(0).values(), *train.parameters(0).values(),
                                 *[m for pair in train.moments(0).values() for m in pair])]
    supports = {k: v.clone() for k, v in train.supports(0).items()}
    for k, v in train.parameters(0).items():
        v.copy_(initial[k])
    for pair in train.moments(0).values():
        for t in pair:
            t.zero_()
    train.steps[0] = 0
    train.step(0, x, gy)
    torch.cuda.synchronize()
    again = [train._gx[:n], *train.gradients(0).values(), *train.parameters(0).values(),
             *[m for pair in train.moments(0).values() for m in pair]]
    assert all(torch.equal(a, b) for a, b in zip(first, again))
    assert all(torch.equal(supports[k], v) for k, v in train.supports(0).items())
    # gate 5: four more steps, each against the closed form from the build's own state
    for k in range(2, 6):
        pre = hidden_major_state(train, layer)
        train.step(0, x, make_gy(case, n, k).to(device))
        post = hidden_major_state(train, layer)
        assert all(np.isfinite(t).all() for s in post.values() for t in s)
        assert _update_errors(pre, post, build_groups(train, layer, n), masks, k) <= GATE3_RELATIVE, k
    assert train.steps[0] == 5


def test_backward_needs_its_forward(device):
    case = synth.CASES["homog_256_1024"]
    runtime = HFFNRuntime([hip_layer(synth.make_layer(case))], device, dense=True)
    train = HFFNTrainRuntime(runtime, **HYPER)
    train.reserve(8)
    x = torch.from_numpy(synth.make_input(case, 8)).to(device)
    gy = make_gy(case, 8, 0).to(device)
    with pytest.raises(RuntimeError, match="must follow"):
        train.backward(0, gy)
    train.forward(0, x, train._z)
    runtime.forward(0, x)  # another forward in between
    with pytest.raises(RuntimeError, match="must follow"):
        train.backward(0, gy)
    train.forward(0, x, train._z)
    with pytest.raises(ValueError, match="N of the forward"):
        train.backward(0, gy[:4].contiguous())
    with pytest.raises(ValueError, match="z must be"):
        train.forward(0, x, torch.empty(10, device=device))
    for pair in ("gemv", "mfma"):  # the planes paths keep no float32 activations: refused, not a KeyError
        runtime.force(pair, pair)
        with pytest.raises(ValueError, match="gather kernels"):
            train.forward(0, x, train._z)
    runtime.force(None, None)


def test_transposed_supports_are_positions_into_the_runtime_arrays(device):
    """The training supports, built on the device by the stable counting sort with slot positions as its payload: up
    slots by input (hidden ascending per input) and down edges by neuron (output ascending per neuron), as positions
    into the runtime's arrays; checked against a brute-force build on a layer with repeated indices in a row and
    neurons without slots."""
    from oracle import transpose
    rng = np.random.default_rng(4)
    d_model, d_ff = 48, 70
    degrees = rng.integers(0, 12, d_ff)
    degrees[::9] = 0
    offsets = np.zeros(d_ff + 1, np.int32)
    offsets[1:] = np.cumsum(degrees)
    up_idx = rng.integers(0, d_model, offsets[-1]).astype(np.int16)
    down_idx = rng.integers(0, d_model, offsets[-1]).astype(np.int16)
    values = lambda size: rng.standard_normal(size).astype(np.float32)  # noqa: E731
    compact = synth.CompactLayer(d_model, d_ff, synth._groups(d_ff), offsets, up_idx, values(up_idx.size), values(d_ff),
                                 offsets, down_idx, values(down_idx.size), values(d_model))
    train = HFFNTrainRuntime(HFFNRuntime([hip_layer(compact)], device, dense=False))
    s = {k: v.cpu().numpy() for k, v in train.supports(0).items()}
    up_owner = owners(compact.up_offsets, compact.d_ff)
    by_input = sorted(range(up_owner.size), key=lambda e: (int(compact.up_idx[e]), e))
    assert s["in_pos"].tolist() == by_input
    assert s["in_hidden"].tolist() == [int(up_owner[e]) for e in by_input]
    assert np.array_equal(s["in_offsets"], np.concatenate([[0], np.cumsum(np.bincount(compact.up_idx, minlength=d_model))]))
    out_offsets, out_hidden, _ = transpose.output_major(d_model, d_ff, compact.down_offsets, compact.down_idx, compact.down_val)
    out_output = owners(out_offsets, d_model)
    by_neuron = sorted(range(out_hidden.size), key=lambda q: (int(out_hidden[q]), q))
    assert s["hid_pos"].tolist() == by_neuron
    assert s["hid_output"].tolist() == [int(out_output[q]) for q in by_neuron]
    assert np.array_equal(s["hid_offsets"], np.concatenate([[0], np.cumsum(np.bincount(out_hidden, minlength=d_ff))]))


@pytest.mark.parametrize("tiled", (False, True))
def test_inference_after_training_reads_the_updated_values(tiled, device):
    """After steps, the runtime's MFMA path (densified planes, rebuilt in place) and its tiles path (the compact rows'
    powers of two, or the tiled stores, rebuilt in place) agree with its gather path."""
    case = synth.Case("mfma_256_1024", 256, 1024, 128, 128, False, 1005)
    layer = synth.make_layer(case)
    runtime = HFFNRuntime([hip_layer(layer)], device, dense=True, tiled=tiled)
    assert runtime.mfma_available
    train = HFFNTrainRuntime(runtime, **dict(HYPER, lr=1e-2))
    n = 256
    x = torch.from_numpy(synth.make_input(case, n)).to(device)
    planes_before = runtime._planes[0]["up"].clone()
    for k in range(3):
        train.step(0, x, make_gy(case, n, k).to(device))
    runtime.force("mfma", "mfma")  # a 256-wide layer takes the register-staged GEMM, which the policy leaves out
    y_mfma = runtime.forward(0, x).clone()
    assert runtime.calls["mfma", "mfma"] == 1
    assert not torch.equal(runtime._planes[0]["up"], planes_before)
    runtime.force("rows", "rows")
    y_rows = runtime.forward(0, x).clone()
    scale = float(y_rows.abs().max())
    assert float((y_mfma - y_rows).abs().max()) <= 1e-5 * max(1.0, scale)
    # the tiles path's tables or stores, rebuilt in place before the decode path next reads them, agree with the gathers
    few = x[:16].contiguous()
    y_few = runtime.forward(0, few).clone()
    runtime.force("tiles", "tiles")
    y_tiles = runtime.forward(0, few).clone()
    assert runtime.calls["tiles", "tiles"] == 1 and not runtime._tiles_stale
    runtime.force(None, None)
    assert float((y_tiles - y_few).abs().max()) <= 1e-5 * max(1.0, float(y_few.abs().max()))
