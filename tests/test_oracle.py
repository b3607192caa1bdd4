"""The oracle, pinned before it is trusted: the reference's known answers, the reference x86 kernel, closed forms,
independent formulations, and planted mistakes that each check must catch. CPU only."""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from hffn_amd import synth
from oracle import reference, transpose, x86_ref

GOLDEN = Path(__file__).resolve().parent / "golden"
ATOL = 2e-5   # runtime/cpu/x86/ffn/inference/hffn/checks.py:17-19, runtime/gpu/nvidia/ffn/inference/checks/parity.py:27
BATCHES = (1, 2, 4, 5, 7, 8, 32, 63, 64, 96, 128, 129)


@pytest.fixture(scope="module")
def test_layers():
    return {name: (synth.make_layer(case), case) for name, case in synth.CASES.items()}


# ------------------------------------------------------------------------------------------- known answers

@pytest.mark.parametrize("name", sorted(synth.CASES))
def test_reference_fingerprints(name, test_layers):
    """The reference's pinned SHA-256 of each test layer and its inputs (runtime/common/ffn/reference/fingerprints.json)."""
    pinned = json.loads((GOLDEN / "fingerprints.json").read_text())["fingerprints"]
    layer, case = test_layers[name]
    assert synth.fingerprint(layer, case) == pinned[name]


def test_fingerprint_detects_a_changed_layer(test_layers):
    """A layer with one value changed is refused (runtime/cpu/x86/ffn/inference/tests/test_layers.py:16-20)."""
    pinned = json.loads((GOLDEN / "fingerprints.json").read_text())["fingerprints"]
    layer, case = test_layers["homog_256_1024"]
    values = layer.up_val.copy()
    values[17] = np.nextafter(values[17], np.float32(1))
    changed = synth.CompactLayer(**{**layer.__dict__, "up_val": values})
    assert synth.fingerprint(changed, case) != pinned["homog_256_1024"]


def test_workload_pins():
    pins = json.loads((GOLDEN / "workloads.json").read_text())
    for name, workload in synth.WORKLOADS.items():
        if workload.d_ff * workload.d_model > 8 * 2**20:
            continue  # the largest layer is pinned by the GPU tests, which generate it anyway
        layer = synth.make_workload_layer(workload)
        assert synth.layer_digest(layer) == pins[name]["layer"], name
        assert layer.up_idx.size == pins[name]["nnz_up"] and layer.down_idx.size == pins[name]["nnz_down"]


def test_reference_batch_chunks():
    """The chunking expectations of runtime/cpu/x86/ffn/inference/tests/test_parity.py:38-42."""
    assert x86_ref.batch_chunks(200, 96) == [(0, 72), (72, 72), (144, 56)]
    assert x86_ref.batch_chunks(128, 96) == [(0, 64), (64, 64)]
    assert x86_ref.batch_chunks(96, 96) == [(0, 96)]


# ------------------------------------------------------------------------------------------------ GELU

def test_erf_libraries_agree():
    z = np.concatenate([np.linspace(-9, 9, 20001), np.geomspace(1e-30, 1e-3, 200), -np.geomspace(1e-30, 1e-3, 200)])
    exact = np.array([math.erf(v) for v in z])
    assert np.max(np.abs(reference._scipy_erf(z) - exact)) <= 4e-16
    half = np.array([math.erf(v * 0.7071067811865476) for v in z])
    assert np.array_equal(reference.gelu_exact(z), 0.5 * z * (1.0 + half))


def test_gelu_special_values():
    z = np.array([0.0, 1.0, -1.0, 3.0, -10.0, 10.0])
    g = reference.gelu_exact(z)
    assert g[0] == 0.0
    assert abs(g[1] - 0.8413447460685429) < 1e-15      # Phi(1) = 0.84134474606854293
    assert abs(g[2] + 0.15865525393145707) < 1e-15     # -(1 - Phi(1))
    assert abs(g[3] - 3 * 0.9986501019683699) < 1e-15  # 3 Phi(3)
    assert abs(g[4]) < 1e-20 and g[5] == 10.0


# ------------------------------------------------------------------------------------------- formulations

@pytest.mark.parametrize("name", sorted(synth.CASES))
def test_three_formulations_agree(name, test_layers):
    layer, case = test_layers[name]
    for n in (1, 3, 64):
        x = synth.make_input(case, n)
        slots = reference.forward_slots(layer, x)
        assert np.max(np.abs(reference.forward_dense(layer, x) - slots)) < 1e-12
        if n <= 3 and layer.d_ff <= 1024:
            assert np.max(np.abs(reference.forward_loops(layer, x) - slots)) < 1e-12


def _full_layer(d_model: int, d_ff: int, seed: int) -> synth.CompactLayer:
    rng = np.random.default_rng(seed)
    offsets = np.arange(d_ff + 1, dtype=np.int32) * d_model
    idx = np.tile(np.arange(d_model, dtype=np.int16), d_ff)
    up = (rng.standard_normal(idx.size) * 0.1).astype(np.float32)
    down = (rng.standard_normal(idx.size) * 0.1).astype(np.float32)
    return synth.CompactLayer(d_model, d_ff, synth._groups(d_ff), offsets, idx, up,
                              (rng.standard_normal(d_ff) * 0.1).astype(np.float32), offsets, idx.copy(), down,
                              (rng.standard_normal(d_model) * 0.1).astype(np.float32))


def test_full_density_is_the_dense_ffn():
    """At 100 % density the HFFN is F.linear -> gelu(approximate="none") -> F.linear (float64 PyTorch),
    with W_up[r, i] = up_val[r * d + i] and W_down[o, r] = down_val[r * d + o]."""
    layer = _full_layer(32, 48, 5)
    x = np.random.default_rng(6).standard_normal((9, 32)).astype(np.float32)
    w_up = torch.from_numpy(layer.up_val.astype(np.float64).reshape(48, 32))
    w_down = torch.from_numpy(layer.down_val.astype(np.float64).reshape(48, 32).T.copy())
    expected = F.linear(F.gelu(F.linear(torch.from_numpy(x).double(), w_up, torch.from_numpy(layer.b_up).double()),
                               approximate="none"), w_down, torch.from_numpy(layer.b_down).double()).numpy()
    for forward in (reference.forward_slots, reference.forward_dense, reference.forward_loops):
        assert np.max(np.abs(forward(layer, x) - expected)) < 1e-12


def test_linearity_of_the_down_side(test_layers):
    """y - b_down is linear in the down values: doubling them doubles y - b_down."""
    layer, case = test_layers["irreg_512_2048"]
    x = synth.make_input(case, 5)
    doubled = synth.CompactLayer(**{**layer.__dict__, "down_val": layer.down_val * np.float32(2)})
    base = reference.forward_slots(layer, x) - layer.b_down.astype(np.float64)
    twice = reference.forward_slots(doubled, x) - layer.b_down.astype(np.float64)
    assert np.max(np.abs(twice - 2 * base)) < 1e-12


# --------------------------------------------------------------------------------- the reference x86 kernel

needs_ref = pytest.mark.skipif(not x86_ref.available(), reason="oracle/_ref not built (make -C oracle)")


@needs_ref
@pytest.mark.parametrize("name", sorted(synth.CASES))
def test_oracle_matches_reference_kernel(name, test_layers):
    """The float64 oracle against the reference x86 AVX2 kernel built from its source: within the reference's
    2e-5 on every route of its parity check (runtime/cpu/x86/ffn/inference/tests/test_parity.py:9-24)."""
    layer, case = test_layers[name]
    kernel = x86_ref.ReferenceKernel(layer, threads=4)
    for n in BATCHES + (200,):
        x = synth.make_input(case, n)
        error = float(np.max(np.abs(kernel.forward(x) - reference.forward(layer, x))))
        assert error <= ATOL, f"{name} N{n}: {error:.3e}"


def _planted(layer, kind: str):
    """A copy of the oracle's input with a plausible mistake planted (the oracle then computes the wrong thing)."""
    if kind == "dropped_up_bias":
        return synth.CompactLayer(**{**layer.__dict__, "b_up": np.zeros_like(layer.b_up)})
    if kind == "dropped_down_bias":
        return synth.CompactLayer(**{**layer.__dict__, "b_down": np.zeros_like(layer.b_down)})
    if kind == "shifted_index":
        return synth.CompactLayer(**{**layer.__dict__, "up_idx": ((layer.up_idx.astype(np.int64) + 1) % layer.d_model).astype(np.int16)})
    if kind == "swapped_sides":
        return synth.CompactLayer(**{**layer.__dict__, "up_val": layer.down_val, "down_val": layer.up_val})
    if kind == "sign":
        return synth.CompactLayer(**{**layer.__dict__, "down_val": -layer.down_val})
    raise ValueError(kind)


@needs_ref
@pytest.mark.parametrize("kind", ["dropped_up_bias", "dropped_down_bias", "shifted_index", "swapped_sides", "sign", "tanh_gelu"])
def test_reference_kernel_catches_planted_oracle_mistakes(kind, test_layers):
    layer, case = test_layers["homog_512_2048"]
    x = synth.make_input(case, 8)
    good = x86_ref.ReferenceKernel(layer, threads=2).forward(x)
    if kind == "tanh_gelu":
        tanh = lambda z: 0.5 * z * (1 + np.tanh(math.sqrt(2 / math.pi) * (z + 0.044715 * z**3)))  # noqa: E731
        wrong = reference.forward_slots(layer, x, gelu=tanh)
    else:
        wrong = reference.forward_slots(_planted(layer, kind), x)
    assert float(np.max(np.abs(good - wrong))) > 10 * ATOL


# ---------------------------------------------------------------------------------------- the transpose

@pytest.mark.parametrize("name", sorted(synth.CASES))
def test_output_major_two_implementations(name, test_layers):
    layer, _ = test_layers[name]
    a = transpose.output_major(layer.d_model, layer.d_ff, layer.down_offsets, layer.down_idx, layer.down_val)
    b = transpose.output_major_loops(layer.d_model, layer.d_ff, layer.down_offsets, layer.down_idx, layer.down_val)
    for left, right in zip(a, b):
        assert left.dtype == right.dtype and np.array_equal(left, right)


@pytest.mark.parametrize("name", sorted(synth.CASES))
def test_output_major_invariants(name, test_layers):
    layer, _ = test_layers[name]
    offsets, hidden, values = transpose.output_major(layer.d_model, layer.d_ff, layer.down_offsets, layer.down_idx, layer.down_val)
    assert offsets[0] == 0 and offsets[-1] == layer.down_idx.size
    assert np.array_equal(np.diff(offsets), np.bincount(layer.down_idx.astype(np.int64), minlength=layer.d_model))
    owner = np.repeat(np.arange(layer.d_ff), np.diff(layer.down_offsets))
    expected = sorted(zip(layer.down_idx.tolist(), owner.tolist(), layer.down_val.view(np.uint32).tolist()))
    output = np.repeat(np.arange(layer.d_model), np.diff(offsets))
    got = sorted(zip(output.tolist(), hidden.tolist(), values.view(np.uint32).tolist()))
    assert got == expected
    for o in range(layer.d_model):
        row = hidden[offsets[o]:offsets[o + 1]].astype(np.int64)
        assert np.all(np.diff(row) > 0)


def test_output_major_duplicates_and_empty_rows():
    """Stable order also when a neuron repeats an output and when neurons and outputs have no slot."""
    offsets = np.array([0, 3, 3, 5, 5], dtype=np.int32)
    idx = np.array([2, 0, 2, 0, 2], dtype=np.int16)
    val = np.arange(5, dtype=np.float32)
    got = transpose.output_major(4, 4, offsets, idx, val)
    assert got[0].tolist() == [0, 2, 2, 5, 5]
    assert got[1].tolist() == [0, 2, 0, 0, 2]
    assert got[2].tolist() == [1.0, 3.0, 0.0, 2.0, 4.0]
    loops = transpose.output_major_loops(4, 4, offsets, idx, val)
    assert all(np.array_equal(a, b) for a, b in zip(got, loops))
