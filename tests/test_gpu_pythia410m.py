"""The full Pythia-410M-architecture model of the HFFN arm on the GPU (24 layers, d_model 1024, 16 heads, rotary on
25 % of the head dimensions, parallel residual, vocab 50304, float32, random init; every FFN an HFFN layer at 50 %
density with uniform per-neuron supports).

* Greedy tokens: 8 prompts x 512 synthetic tokens then 128 greedy decode steps; every HFFN token is explained by the
  dense float32 arm or the float64 arbiter (``runtime/common/pythia/hffn_pythia/parity_model.py:104-118``), and the
  predeclared negative control (layer 3 ``attention.dense.weight`` x 1.5) is caught.
* Every exported layer through the leaf's runtime, at the reference's token counts, with the policy and every forced
  kernel pair: same bits on repeat and max |y - y64| / max(1, |y64|) <= 1e-5 against the float64 oracle
  (``runtime/gpu/nvidia/llm/inference/checks/parity_layers.py:28-61``; the tolerance is the stated fp32 bound).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hffn_amd import parity, pythia, pythia_check, synth
from oracle import reference

pytestmark = pytest.mark.gpu

LAYERS = 24
BATCHES = (1, 2, 4, 5, 32, 63, 64, 128, 129, 256, 512)  # parity_layers.py:28


@pytest.fixture(scope="module")
def assets(tmp_path_factory):
    root = tmp_path_factory.mktemp("pythia410m")
    pythia.write_random_pythia(root / "model", root / "export", density=0.5, seed=104)
    print(f"pythia410m: random-init checkpoint and {LAYERS} exports written", flush=True)
    return root / "model", root / "export"


@pytest.fixture(scope="module")
def arms(assets, device):
    model_dir, export_dir = assets
    dense = pythia.load_pythia(model_dir, export_dir, "dense", device)
    hffn = pythia.load_pythia(model_dir, export_dir, "hffn", device)
    arbiter = pythia.load_pythia(model_dir, export_dir, "dense", device).double()
    assert dense.config.num_hidden_layers == LAYERS and dense.config.vocab_size == 50304
    prompts = [pythia.synthetic_prompts(8, 512, 50304).to(device)]
    return dense, hffn, arbiter, prompts


def test_pythia410m_greedy_tokens(arms):
    dense, hffn, arbiter, prompts = arms
    print("pythia410m: 8 x 512 prompt, 128 greedy steps", flush=True)
    report = pythia_check.check_arm(dense, hffn, arbiter, prompts, 128, log=lambda s: print(s, flush=True))
    assert report["tokens"] == 8 * (512 + 128)
    assert report["unexplained"] == 0, report
    calls = hffn.hffn_runtime.calls
    assert sum(calls.values()) == LAYERS * (1 + 128)  # one prefill call and one call per decode step, per layer


def test_pythia410m_negative_control(assets, arms, device):
    dense, _, arbiter, prompts = arms
    faulty = pythia.load_pythia(*assets, "hffn", device)
    pythia_check.inject_fault(faulty, layer=pythia_check.FAULT_LAYER)
    report = pythia_check.check_arm(dense, faulty, arbiter, prompts, 128, log=lambda s: print(s, flush=True))
    assert report["unexplained"] > 0, report


@pytest.fixture(scope="module")
def leaf_runtime(assets, device):
    _, export_dir = assets
    layers = pythia.read_layers(export_dir, LAYERS)
    return layers, pythia.hip_runtime(layers, device)


def _compact(layer: dict) -> synth.CompactLayer:
    n = lambda key: layer[key].numpy()  # noqa: E731
    return synth.CompactLayer(layer["d_model"], layer["d_ff"], np.zeros(5, np.int32), n("up_row_offsets"), n("up_idx"),
                              n("up_val"), n("b_up"), n("down_row_offsets"), n("down_idx"), n("down_val"), n("b_down"))


@pytest.mark.parametrize("index", range(LAYERS))
def test_pythia410m_export_layer_parity(index, leaf_runtime, device):
    layers, runtime = leaf_runtime
    compact = _compact(layers[index])
    weights = reference.dense_weights(compact)
    generator = np.random.default_rng([1040, index])
    worst = {}
    for n in BATCHES:
        x = generator.standard_normal((n, compact.d_model)).astype(np.float32)
        expected = torch.from_numpy(reference.forward_dense(compact, x, weights)).to(device)
        result = parity.check(runtime, index, torch.from_numpy(x).to(device), expected)
        assert result.repeatable and result.sequential_bits, f"layer {index} N{n}: bits differ on repeat"
        worst[n] = result.relative
        assert result.relative <= 1e-5, (index, n, result.pairs)
    print(f"layer {index}: max relative " + " ".join(f"N{n}={e:.1e}" for n, e in worst.items()), flush=True)
