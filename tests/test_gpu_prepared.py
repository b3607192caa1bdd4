"""The decode launch path (``PreparedRuntime``, plans of the C ABI) on the GPU: bit-identical to ``HFFNRuntime`` on
every gather pair, the decode GEMVs, the compact-store MFMA path and every token count it serves, the same ``calls`` bookkeeping, plans released when the work buffers move
or a mode is forced, and the float64 oracle on the reference test layers (2e-5 absolute, as
runtime/gpu/nvidia/ffn/inference/checks/parity.py:26-61)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hffn_amd import synth
from hffn_amd.ffn import hip_layer
from hffn_amd.prepared_runtime import PreparedRuntime
from hffn_amd.runtime import HFFNRuntime
from oracle import reference

pytestmark = pytest.mark.gpu

ATOL = 2e-5
TOKENS = (1, 2, 3, 4, 5, 8, 9, 16, 32, 33, 64, 128)


@pytest.fixture(scope="module")
def runtimes(device):
    out = {}
    for name, case in synth.CASES.items():
        compact = synth.make_layer(case)
        layers = [hip_layer(compact)]
        out[name] = (compact, case, HFFNRuntime(layers, device, dense=True), PreparedRuntime(layers, device, dense=True))
    return out


@pytest.mark.parametrize("name", sorted(synth.CASES))
def test_prepared_matches_control_bitwise(name, runtimes):
    compact, case, control, prepared = runtimes[name]
    for n in TOKENS:
        x = torch.from_numpy(synth.make_input(case, n)).to(control.device)
        expected = control.forward(0, x).clone()
        for repeat in range(2):  # the second call runs from the plan the first one built
            got = prepared.forward(0, x)
            assert torch.equal(got, expected), (name, n, repeat)
        assert prepared.modes(n) == control.modes(n)
        oracle_y = reference.forward(compact, x.double().cpu().numpy())
        assert float((got.double().cpu() - torch.from_numpy(oracle_y)).abs().max()) <= ATOL, (name, n)


@pytest.mark.parametrize("pair", [("edges", "edges"), ("edges", "rows"), ("rows", "edges"), ("rows", "rows"),
                                  ("gemv", "gemv"), ("tiles", "tiles")])
def test_prepared_forced_pairs(pair, runtimes, device):
    compact, case, control, prepared = runtimes["irreg_512_2048"]
    try:
        control.force(*pair)
        prepared.force(*pair)
        for n in ((1, 4, 7, 24, 33) if pair[0] in ("gemv", "tiles") else (1, 4, 7, 64)):
            x = torch.from_numpy(synth.make_input(case, n)).to(device)
            assert torch.equal(prepared.forward(0, x), control.forward(0, x)), (pair, n)
            assert prepared._plans[(0, n)][1:] == pair
    finally:
        control.force(None, None)
        prepared.force(None, None)
    assert prepared._plans == {}


@pytest.mark.parametrize("name", ["irreg_512_2048", "homog_256_1024"])
def test_prepared_tiles_on_the_tiled_store(name, runtimes, device):
    """With tiled=True the planned launches (hffn_plan_tiles) read the tiled copies: bit-identical to the eager calls of
    a tiled runtime and to the default runtime's calls on the compact rows (one block shape, the same tiles), and the
    plans see the copies rebuilt after an update of the compact values."""
    compact, case, control, _ = runtimes[name]
    tiled_control = HFFNRuntime([hip_layer(compact)], device, tiled=True)
    tiled_prepared = PreparedRuntime([hip_layer(compact)], device, tiled=True)
    for runtime in (control, tiled_control, tiled_prepared):
        runtime.force("tiles", "tiles")
    try:
        for n in (1, 4, 7, 24, 33, 64):
            x = torch.from_numpy(synth.make_input(case, n)).to(device)
            expected = control.forward(0, x).clone()
            assert torch.equal(tiled_control.forward(0, x), expected), (name, n)
            for repeat in range(2):  # the second call runs from the plan the first one built
                assert torch.equal(tiled_prepared.forward(0, x), expected), (name, n, repeat)
            assert tiled_prepared._plans[(0, n)][1:] == ("tiles", "tiles")
        x = torch.from_numpy(synth.make_input(case, 16)).to(device)
        before = tiled_prepared.forward(0, x).clone()
        for runtime in (tiled_control, tiled_prepared):
            runtime._tensors[0]["up_val"].mul_(0.5)
            runtime.invalidate_planes(0)  # marks the tiled copies stale as well
        after = tiled_prepared.forward(0, x).clone()  # launched from the plan made before the update
        assert torch.equal(after, tiled_control.forward(0, x))
        assert not torch.equal(after, before)
    finally:
        for runtime in (control, tiled_control, tiled_prepared):
            runtime.force(None, None)


def test_plans_follow_the_buffers(device):
    """A larger N reallocates the work buffers: the plans made before are released and rebuilt on the new buffers;
    the calls counter counts plan launches like control calls; an input that is a row-offset view works."""
    case = synth.CASES["homog_256_1024"]
    layers = [hip_layer(synth.make_layer(case))]
    control, prepared = HFFNRuntime(layers, device, dense=True), PreparedRuntime(layers, device, dense=True)
    x1 = torch.from_numpy(synth.make_input(case, 1)).to(device)
    x8 = torch.from_numpy(synth.make_input(case, 8)).to(device)
    y1 = control.forward(0, x1).clone()
    y8 = control.forward(0, x8).clone()
    assert torch.equal(prepared.forward(0, x1), y1)
    assert set(prepared._plans) == {(0, 1)}
    assert torch.equal(prepared.forward(0, x8), y8)
    assert set(prepared._plans) == {(0, 8)}  # the n=1 plan went with the old buffers
    assert torch.equal(prepared.forward(0, x1), y1)
    assert torch.equal(control.forward(0, x1), y1)
    assert prepared.calls == control.calls
    block = torch.from_numpy(synth.make_input(case, 6)).to(device)
    view = block[2:5]  # a contiguous view at a row offset
    assert torch.equal(prepared.forward(0, view), control.forward(0, view.clone()))


def test_prepared_refuses_what_the_control_refuses(device):
    case = synth.CASES["homog_256_1024"]
    prepared = PreparedRuntime([hip_layer(synth.make_layer(case))], device, dense=True)
    with pytest.raises(ValueError, match="contiguous float32"):
        prepared.forward(0, torch.zeros(2, case.d_model + 1, device=device))
    with pytest.raises(ValueError, match="contiguous float32"):
        prepared.forward(0, torch.zeros(2, case.d_model, device=device, dtype=torch.float64))
    with pytest.raises(ValueError, match="unsupported token count"):
        prepared.forward(0, torch.zeros(0, case.d_model, device=device))
    with pytest.raises(IndexError):
        prepared.forward(3, torch.zeros(1, case.d_model, device=device))
    assert np.isfinite(prepared.forward(0, torch.ones(1, case.d_model, device=device)).cpu().numpy()).all()


def test_gemv_plans_see_updated_values(device):
    """A GEMV plan bakes the layer's plane pointers; after a training-style update of the compact values (in place,
    then invalidate_planes) the planned launch rebuilds the planes first and matches the control bit for bit."""
    case = synth.CASES["homog_512_2048"]
    compact = synth.make_layer(case)
    control, prepared = HFFNRuntime([hip_layer(compact)], device, dense=True), PreparedRuntime([hip_layer(compact)], device, dense=True)
    control.force("gemv", "gemv")
    prepared.force("gemv", "gemv")
    x = torch.from_numpy(synth.make_input(case, 16)).to(device)
    before = control.forward(0, x).clone()
    assert torch.equal(prepared.forward(0, x), before)
    assert (0, 16) in prepared._plans
    for runtime in (control, prepared):
        runtime._tensors[0]["up_val"].mul_(0.5)
        runtime.invalidate_planes(0)
    after = prepared.forward(0, x).clone()  # launched from the plan made before the update
    assert torch.equal(after, control.forward(0, x))
    assert not torch.equal(after, before)
