"""The Pythia arm on the GPU: random-init GPT-NeoX models whose FFNs run through the HFFN HIP runtime, checked
token by token against the dense float32 arm and the float64 arbiter (``runtime/common/pythia/hffn_pythia/
parity_model.py:95-126``), with the predeclared negative control that must be caught."""
from __future__ import annotations

import pytest
import torch

from hffn_amd import pythia, pythia_check

pytestmark = pytest.mark.gpu

SHAPES = {
    # Gather kernels only (d_model 64 has no MFMA tiling): prefill 2x16 and decode 2 tokens per call.
    "tiny": dict(num_hidden_layers=2, hidden_size=64, num_attention_heads=4, intermediate_size=256, vocab_size=500),
    # MFMA prefill (2x64 tokens per call, on the streamed GEMM) and edges decode, 4 blocks of the Pythia layout at the
    # 70M widths.
    "narrow": dict(num_hidden_layers=4, hidden_size=512, num_attention_heads=8, intermediate_size=2048, vocab_size=2000),
}


@pytest.fixture(scope="module", params=sorted(SHAPES))
def arms(request, tmp_path_factory, device):
    shape = SHAPES[request.param]
    root = tmp_path_factory.mktemp(request.param)
    pythia.write_random_pythia(root / "model", root / "export", seed=11, **shape)
    load = lambda ffn: pythia.load_pythia(root / "model", root / "export", ffn, device)  # noqa: E731
    length = 16 if request.param == "tiny" else 64
    prompts = [pythia.synthetic_prompts(2, length, shape["vocab_size"]).to(device)]
    return request.param, load, prompts


def test_hffn_arm_tokens(arms):
    name, load, prompts = arms
    dense, hffn, arbiter = load("dense"), load("hffn"), load("dense").double()
    print(f"pythia {name}: prefill {tuple(prompts[0].shape)}, 24 decode steps", flush=True)
    totals = pythia_check.check_arm(dense, hffn, arbiter, prompts, 24, log=lambda s: print(s, flush=True))
    assert totals["unexplained"] == 0, totals
    assert totals["prefill_max_dlogit"] < 1e-3, totals
    modes = {key for key in hffn.hffn_runtime.calls}
    assert ("edges", "edges") in modes
    if name == "narrow":
        assert ("mfma", "mfma") in modes


def test_negative_control_is_caught(arms):
    name, load, prompts = arms
    dense, faulty, arbiter = load("dense"), load("hffn"), load("dense").double()
    pythia_check.inject_fault(faulty, layer=1)
    totals = pythia_check.check_arm(dense, faulty, arbiter, prompts, 24, log=lambda s: print(s, flush=True))
    assert totals["unexplained"] > 0, totals
