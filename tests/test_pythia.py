"""The Pythia arm's host side, on the CPU: the export format and its validation, the dense arm's FFN against the
float64 oracle, the loader's wiring of the HFFN hook (with a dense stand-in runtime), and the token criterion
(``runtime/common/pythia/hffn_pythia/parity_model.py``) with its negative control."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from hffn_amd import pythia, pythia_check, synth
from oracle import reference

TINY = dict(num_hidden_layers=2, hidden_size=64, num_attention_heads=4, intermediate_size=256, vocab_size=500)


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    root = tmp_path_factory.mktemp("pythia")
    pythia.write_random_pythia(root / "model", root / "export", seed=7, **TINY)
    return root / "model", root / "export"


class DenseStandIn:
    """A CPU stand-in of the HFFN runtime for wiring tests: the export's FFN with torch dense ops."""

    def __init__(self, layers):
        self.layers = layers
        self.calls = 0

    def forward(self, index, x):
        layer = self.layers[index]
        w_up = torch.zeros(layer["d_ff"], layer["d_model"])
        w_up[pythia.hidden_of_slot(layer, "up"), layer["up_idx"].long()] = layer["up_val"]
        w_down = torch.zeros(layer["d_model"], layer["d_ff"])
        w_down[layer["down_idx"].long(), pythia.hidden_of_slot(layer, "down")] = layer["down_val"]
        self.calls += 1
        return F.linear(F.gelu(F.linear(x, w_up, layer["b_up"]), approximate="none"), w_down, layer["b_down"])


def test_export_round_trip(tmp_path):
    compact = synth.make_layer(synth.CASES["irreg_512_2048"])
    path = pythia.layer_path(tmp_path, 0)
    pythia.write_layer(path, pythia.export_of_compact(compact))
    layer = pythia.read_layer(path, groups=True)
    assert layer["d_model"] == 512 and layer["d_ff"] == 2048
    for name, field in (("up_row_offsets", "up_offsets"), ("up_idx", "up_idx"), ("up_val", "up_val"), ("b_up", "b_up"),
                        ("down_row_offsets", "down_offsets"), ("down_idx", "down_idx"), ("down_val", "down_val"),
                        ("b_down", "b_down"), ("group_hidden_offsets", "groups")):
        assert np.array_equal(layer[name].numpy(), getattr(compact, field)), name
    assert torch.equal(pythia.hidden_of_slot(layer, "down"),
                       torch.from_numpy(np.repeat(np.arange(2048), np.diff(compact.down_offsets))))


@pytest.mark.parametrize("fault", ["format", "dtype", "offsets", "index", "bias", "groups"])
def test_export_validation(fault, tmp_path):
    """The reader refuses what ``export.py:29-41`` refuses."""
    compact = synth.make_layer(synth.CASES["homog_256_1024"])
    raw = {"format": pythia.FORMAT, "d_model": 256, "d_ff": 1024, **{k: v.clone() for k, v in pythia.export_of_compact(compact).items()
                                                                     if isinstance(v, torch.Tensor)}}
    if fault == "format":
        raw["format"] = "something_else"
    elif fault == "dtype":
        raw["up_val"] = raw["up_val"].double()
    elif fault == "offsets":
        raw["down_row_offsets"][3] = raw["down_row_offsets"][4] + 1
    elif fault == "index":
        raw["up_idx"][5] = 256
    elif fault == "bias":
        raw["b_down"] = raw["b_down"][:-1]
    elif fault == "groups":
        raw["group_hidden_offsets"] = torch.tensor([0, 10, 5, 900, 1024], dtype=torch.int32)
    path = tmp_path / "bad.pt"
    torch.save(raw, path)
    with pytest.raises(ValueError):
        pythia.read_layer(path, groups=True)


def test_config_is_pythia_410m_shaped():
    config = pythia.pythia_config()
    assert (config.hidden_size, config.num_hidden_layers, config.num_attention_heads, config.intermediate_size,
            config.vocab_size) == (1024, 24, 16, 4096, 50304)
    assert config.use_parallel_residual and config.hidden_act == "gelu"
    assert config.rope_parameters["partial_rotary_factor"] == 0.25


def test_dense_arm_ffn_is_the_oracle(tiny):
    """The dense arm's GPTNeoXMLP, with its weights set from the export on the support, computes the float64 oracle's
    FFN of the same layer (to float32 accuracy)."""
    model_dir, export_dir = tiny
    model = pythia.load_pythia(model_dir, export_dir, "dense", "cpu")
    assert model.hffn_runtime is None
    layer = pythia.read_layer(pythia.layer_path(export_dir, 1))
    compact = synth.CompactLayer(layer["d_model"], layer["d_ff"], np.zeros(5, np.int32), layer["up_row_offsets"].numpy(),
                                 layer["up_idx"].numpy(), layer["up_val"].numpy(), layer["b_up"].numpy(),
                                 layer["down_row_offsets"].numpy(), layer["down_idx"].numpy(), layer["down_val"].numpy(),
                                 layer["b_down"].numpy())
    x = torch.randn(7, layer["d_model"], generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        y = model.gpt_neox.layers[1].mlp(x)
    assert float((y.double() - torch.from_numpy(reference.forward(compact, x.numpy()))).abs().max()) < 1e-5


def test_hffn_arm_wiring(tiny):
    """The HFFN arm allocates no dense FFN, routes every block's FFN through the runtime and gives the dense arm's
    logits."""
    model_dir, export_dir = tiny
    dense = pythia.load_pythia(model_dir, export_dir, "dense", "cpu")
    hffn = pythia.load_pythia(model_dir, export_dir, "hffn", "cpu", make_runtime=DenseStandIn)
    assert not any(".mlp." in name for name, _ in hffn.named_parameters())
    assert all(isinstance(block.mlp, pythia.HFFNMLP) for block in hffn.gpt_neox.layers)
    prompt = pythia.synthetic_prompts(2, 12, 500)
    with torch.no_grad():
        a, b = dense(input_ids=prompt).logits, hffn(input_ids=prompt).logits
    assert hffn.hffn_runtime.calls == TINY["num_hidden_layers"]
    assert float((a - b).abs().max()) < 1e-5


def test_token_check_and_negative_control(tiny):
    model_dir, export_dir = tiny
    dense = pythia.load_pythia(model_dir, export_dir, "dense", "cpu")
    arbiter = pythia.load_pythia(model_dir, export_dir, "dense", "cpu").double()
    hffn = pythia.load_pythia(model_dir, export_dir, "hffn", "cpu", make_runtime=DenseStandIn)
    prompts = [pythia.synthetic_prompts(2, 16, 500)]
    quiet = lambda _: None  # noqa: E731
    assert pythia_check.check_arm(dense, hffn, arbiter, prompts, 6, log=quiet)["unexplained"] == 0
    faulty = pythia.load_pythia(model_dir, export_dir, "hffn", "cpu", make_runtime=DenseStandIn)
    pythia_check.inject_fault(faulty, layer=1)
    assert pythia_check.check_arm(dense, faulty, arbiter, prompts, 6, log=quiet)["unexplained"] > 0


def test_loader_refuses_unknown_arm(tiny):
    with pytest.raises(ValueError, match="dense"):
        pythia.load_pythia(*tiny, "sparse", "cpu")
