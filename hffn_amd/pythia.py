"""Pythia (GPT-NeoX) with its FFNs executed dense or by the HFFN HIP runtime: the two-arm loader, its hook, the
compact export format, and a writer of random-init Pythia-shaped checkpoints with synthetic exports.

Drop-in for the reference's shared Pythia level and its NVIDIA leaf:

* ``load_pythia(model_dir, export_dir, ffn, device="cuda", make_runtime=None)`` — both
  ``runtime/gpu/nvidia/llm/inference/hffn_pythia_cuda/model.py:23-28`` (leaf: the HIP runtime is built by default)
  and ``runtime/common/pythia/hffn_pythia/model.py:82-111`` (shared: ``make_runtime(layers)`` given);
* ``HFFNMLP(runtime, index)`` — ``model.py:27-37``: replaces ``block.mlp``; its output is a view of the runtime's
  output buffer, consumed by the block's residual sum before the next FFN call;
* ``layer_from_export(layer)`` — ``hffn_pythia_cuda/model.py:11-15``;
* ``read_layer``/``read_layers``/``hidden_of_slot`` — ``runtime/common/pythia/hffn_pythia/export.py:13-57``, the
  ``hffn_training_compact_g4_v2`` format, with its validation; ``write_layer`` writes the same format.

Both arms build the same GPT-NeoX model, load the same non-FFN tensors from ``model_dir/model.safetensors`` and read
the FFNs from the same export: the dense arm sets ``GPTNeoXMLP`` weights on the fixed support (zeros elsewhere), the
HFFN arm never allocates a dense FFN and hands the activations to the runtime. Embeddings, attention (PyTorch SDPA),
LayerNorm, KV cache and head stay PyTorch.
"""
from __future__ import annotations

from contextlib import contextmanager
from pathlib import Path

import numpy as np
import torch
from torch import nn

FORMAT = "hffn_training_compact_g4_v2"
_TYPES = {
    "up_row_offsets": torch.int32, "up_idx": torch.int16, "up_val": torch.float32, "b_up": torch.float32,
    "down_row_offsets": torch.int32, "down_idx": torch.int16, "down_val": torch.float32, "b_down": torch.float32,
}
# Buffers of older GPT-NeoX checkpoints that the model classes rebuild themselves.
_LEGACY = (".attention.bias", ".attention.masked_bias", ".attention.rotary_emb.inv_freq")


# ------------------------------------------------------------------------------------------------- export format

def read_layer(path: str | Path, *, groups: bool = False) -> dict:
    """The validated arrays of one export file, as contiguous CPU tensors (``export.py:20-48``). With ``groups``,
    also ``group_hidden_offsets`` (int32[5], 0 .. d_ff, monotonic)."""
    path = Path(path)
    raw = torch.load(path, map_location="cpu", weights_only=True)
    if raw.get("format") != FORMAT:
        raise ValueError(f"{path}: expected a {FORMAT} export")
    layer: dict = {"d_model": int(raw["d_model"]), "d_ff": int(raw["d_ff"])}
    for name, dtype in _TYPES.items():
        if raw[name].dtype != dtype:
            raise ValueError(f"{path}: {name} must be {dtype}")
        layer[name] = raw[name].contiguous()
    h, f = layer["d_model"], layer["d_ff"]
    if layer["b_up"].numel() != f or layer["b_down"].numel() != h:
        raise ValueError(f"{path}: bias dimensions do not match d_model/d_ff")
    for side in ("up", "down"):
        offsets, index, values = layer[f"{side}_row_offsets"], layer[f"{side}_idx"], layer[f"{side}_val"]
        if offsets.numel() != f + 1 or int(offsets[0]) != 0 or int(offsets[-1]) != values.numel() or index.numel() != values.numel():
            raise ValueError(f"{path}: invalid {side} hidden-major storage")
        if bool((offsets.diff() < 0).any()) or (index.numel() and (int(index.min()) < 0 or int(index.max()) >= h)):
            raise ValueError(f"{path}: invalid {side} offsets or feature index")
    if groups:
        partition = raw["group_hidden_offsets"]
        if partition.dtype != torch.int32 or tuple(partition.shape) != (5,) or int(partition[0]) != 0 \
                or int(partition[-1]) != f or bool((partition.diff() < 0).any()):
            raise ValueError(f"{path}: invalid group_hidden_offsets")
        layer["group_hidden_offsets"] = partition.contiguous()
    return layer


def layer_path(export_dir: str | Path, index: int) -> Path:
    return Path(export_dir) / f"layer{index}" / f"{FORMAT}.pt"


def read_layers(export_dir: str | Path, count: int) -> list[dict]:
    return [read_layer(layer_path(export_dir, index)) for index in range(count)]


def write_layer(path: str | Path, layer: dict) -> None:
    """Write one export file in the ``hffn_training_compact_g4_v2`` format (readable by ``read_layer``)."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    f = int(layer["d_ff"])
    raw = {"format": FORMAT, "d_model": int(layer["d_model"]), "d_ff": f,
           "group_hidden_offsets": layer.get("group_hidden_offsets",
                                             torch.tensor([(g * f) // 4 for g in range(5)], dtype=torch.int32))}
    for name, dtype in _TYPES.items():
        raw[name] = layer[name].to(dtype).contiguous()
    torch.save(raw, path)


def hidden_of_slot(layer: dict, side: str) -> torch.Tensor:
    """Hidden neuron owning each compact slot of one side (int64[nnz])."""
    return torch.repeat_interleave(torch.arange(layer["d_ff"]), layer[f"{side}_row_offsets"].diff().long())


def export_of_compact(compact) -> dict:
    """The export dict of a compact hidden-major layer (``hffn_amd.synth.CompactLayer``)."""
    t = torch.from_numpy
    return {"d_model": compact.d_model, "d_ff": compact.d_ff, "up_row_offsets": t(compact.up_offsets),
            "up_idx": t(compact.up_idx), "up_val": t(compact.up_val), "b_up": t(compact.b_up),
            "down_row_offsets": t(compact.down_offsets), "down_idx": t(compact.down_idx),
            "down_val": t(compact.down_val), "b_down": t(compact.b_down),
            "group_hidden_offsets": t(compact.groups)}


# ----------------------------------------------------------------------------------------------------- the hook

class HFFNMLP(nn.Module):
    """Replacement of ``block.mlp``. Its output is a view of the runtime's output buffer, which the block consumes
    (residual sum) before the next FFN call overwrites it."""

    def __init__(self, runtime, index: int) -> None:
        super().__init__()
        self.runtime, self.index = runtime, index

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        shape = hidden_states.shape
        return self.runtime.forward(self.index, hidden_states.reshape(-1, shape[-1])).view(shape)


def layer_from_export(layer: dict, device: str | torch.device | None = None):
    """The ``HFFNLayer`` of one export layer (``read_layer``); the output-major store is built on the device."""
    from .runtime import HFFNLayer
    return HFFNLayer.from_hidden_major(layer["d_model"], layer["d_ff"], layer["b_up"], layer["up_row_offsets"],
                                       layer["up_idx"], layer["up_val"], layer["b_down"], layer["down_row_offsets"],
                                       layer["down_idx"], layer["down_val"], device=device)


def hip_runtime(layers: list[dict], device: str | torch.device = "cuda"):
    """The HFFN HIP runtime of a model's export layers: ``PreparedRuntime`` (decode calls launched from per-(layer, N)
    plans), as the reference leaf's ``_runtime`` (``runtime/gpu/nvidia/llm/inference/hffn_pythia_cuda/model.py:18-20``)."""
    from .prepared_runtime import PreparedRuntime
    return PreparedRuntime([layer_from_export(layer, device) for layer in layers], device)


# --------------------------------------------------------------------------------------------------- the loader

@torch.no_grad()
def _set_dense_mlp(mlp: nn.Module, layer: dict) -> None:
    up, down = mlp.dense_h_to_4h, mlp.dense_4h_to_h
    if tuple(up.weight.shape) != (layer["d_ff"], layer["d_model"]):
        raise ValueError("export and model dimensions differ")
    up.weight.zero_()
    up.weight[hidden_of_slot(layer, "up"), layer["up_idx"].long()] = layer["up_val"].to(up.weight.dtype)
    up.bias.copy_(layer["b_up"])
    down.weight.zero_()
    down.weight[layer["down_idx"].long(), hidden_of_slot(layer, "down")] = layer["down_val"].to(down.weight.dtype)
    down.bias.copy_(layer["b_down"])


@torch.no_grad()
def _load_non_ffn(model: nn.Module, checkpoint: Path) -> None:
    from safetensors import safe_open
    targets = {name: tensor for name, tensor in model.state_dict().items() if ".mlp." not in name}
    with safe_open(str(checkpoint), framework="pt", device="cpu") as source:
        names = [name for name in source.keys() if ".mlp." not in name and (name in targets or not name.endswith(_LEGACY))]
        if set(names) != set(targets):
            raise ValueError(f"checkpoint and model tensors differ: {sorted(set(names) ^ set(targets))}")
        for name in names:
            targets[name].copy_(source.get_tensor(name))


class _NoFFN(nn.Module):
    """Parameterless stand-in for ``GPTNeoXMLP`` while the HFFN arm is built: no dense FFN is allocated (nor
    initialised); ``HFFNMLP`` takes its place before the model is used."""

    def __init__(self, config):
        super().__init__()


@contextmanager
def without_dense_ffn():
    from transformers.models.gpt_neox import modeling_gpt_neox
    original = modeling_gpt_neox.GPTNeoXMLP
    modeling_gpt_neox.GPTNeoXMLP = _NoFFN
    try:
        yield
    finally:
        modeling_gpt_neox.GPTNeoXMLP = original


def load_pythia(model_dir: str | Path, export_dir: str | Path, ffn: str, device: str | torch.device = "cuda",
                make_runtime=None) -> nn.Module:
    """Pythia in eval mode (float32, on ``device``) with its FFNs from ``export_dir``, executed dense or by HFFN.

    ``make_runtime(layers)`` builds the HFFN runtime from the export layers (default: the HIP runtime on ``device``);
    it is called for the HFFN arm only, so the dense arm needs no GPU kernel. The HFFN arm exposes its runtime as
    ``model.hffn_runtime`` (None in the dense arm)."""
    from transformers import AutoConfig, AutoModelForCausalLM
    if ffn not in ("dense", "hffn"):
        raise ValueError("ffn must be 'dense' or 'hffn'")
    config = AutoConfig.from_pretrained(str(model_dir))
    if ffn == "hffn":
        with without_dense_ffn():
            model = AutoModelForCausalLM.from_config(config, dtype=torch.float32)
        assert not any(".mlp." in name for name, _ in model.named_parameters())
    else:
        model = AutoModelForCausalLM.from_config(config, dtype=torch.float32)
    _load_non_ffn(model, Path(model_dir) / "model.safetensors")
    blocks = model.gpt_neox.layers
    layers = read_layers(export_dir, len(blocks))
    runtime = None
    if ffn == "dense":
        for block, layer in zip(blocks, layers):
            _set_dense_mlp(block.mlp, layer)
    else:
        runtime = (make_runtime or (lambda ls: hip_runtime(ls, device)))(layers)
        for index, block in enumerate(blocks):
            block.mlp = HFFNMLP(runtime, index)
    model = model.to(device).eval().requires_grad_(False)
    model.hffn_runtime = runtime
    return model


# ------------------------------------------------------------------------------ random-init Pythia-shaped models

PYTHIA_410M = dict(hidden_size=1024, num_hidden_layers=24, num_attention_heads=16, intermediate_size=4096,
                   vocab_size=50304, max_position_embeddings=2048, rotary_pct=0.25, rotary_emb_base=10000,
                   use_parallel_residual=True, layer_norm_eps=1e-5, hidden_act="gelu", tie_word_embeddings=False)


def pythia_config(**overrides):
    """A ``GPTNeoXConfig`` of the Pythia family (Pythia-410M by default): parallel attention + MLP residual, rotary
    on 25 % of the head dimensions, exact-erf GELU."""
    from transformers import GPTNeoXConfig
    values = {**PYTHIA_410M, **overrides}
    rotary = values.pop("rotary_pct")
    base = values.pop("rotary_emb_base")
    config = GPTNeoXConfig(**values)
    config.rope_parameters = {"rope_theta": float(base), "partial_rotary_factor": float(rotary), "rope_type": "default"}
    config.architectures = ["GPTNeoXForCausalLM"]
    return config


def write_random_checkpoint(model_dir: str | Path, seed: int = 104, **config_overrides):
    """Write a random-init Pythia-shaped checkpoint: ``config.json`` + ``model.safetensors`` of the non-FFN tensors,
    initialised by the model class from ``torch.manual_seed(seed)``. Returns the config."""
    from safetensors.torch import save_file
    from transformers import AutoModelForCausalLM
    config = pythia_config(**config_overrides)
    model_dir = Path(model_dir)
    model_dir.mkdir(parents=True, exist_ok=True)
    config.save_pretrained(str(model_dir))
    torch.manual_seed(seed)
    with without_dense_ffn():
        model = AutoModelForCausalLM.from_config(config, dtype=torch.float32)
    state = {name: tensor.contiguous() for name, tensor in model.state_dict().items() if ".mlp." not in name}
    save_file(state, str(model_dir / "model.safetensors"))
    return config


def write_random_exports(export_dir: str | Path, config, density: float = 0.5, seed: int = 104) -> None:
    """One export per layer of ``config``: every neuron's up and down supports are ``round(density * d_model)``
    indices drawn uniformly without replacement and sorted, values ~N(0, initializer_range), biases zero (layer l
    draws from seed ``seed * 100 + l``)."""
    from .synth import Workload, make_workload_layer
    d, f = config.hidden_size, config.intermediate_size
    degree = max(1, int(round(density * d)))
    for index in range(config.num_hidden_layers):
        workload = Workload(f"pythia_layer{index}", d, f, degree, seed * 100 + index, w_std=config.initializer_range)
        write_layer(layer_path(export_dir, index), export_of_compact(make_workload_layer(workload)))


def write_random_pythia(model_dir: str | Path, export_dir: str | Path, density: float = 0.5, seed: int = 104,
                        **config_overrides) -> None:
    """A random-init checkpoint (``write_random_checkpoint``) and its exports at one density
    (``write_random_exports``)."""
    config = write_random_checkpoint(model_dir, seed, **config_overrides)
    write_random_exports(export_dir, config, density, seed)


@torch.no_grad()
def share_non_ffn(model: nn.Module, source: nn.Module) -> None:
    """Make ``model`` read the non-FFN parameters of ``source`` (both loaded from the same checkpoint) instead of its
    own copy, so that two arms in one process differ by their FFNs only (``runtime/common/pythia/hffn_pythia/
    model.py:114-124``)."""
    owned = dict(source.named_parameters())
    for prefix, module in model.named_modules():
        for key, parameter in list(module._parameters.items()):
            name = f"{prefix}.{key}" if prefix else key
            if parameter is not None and ".mlp." not in name:
                module._parameters[key] = owned[name]


def synthetic_prompts(batch: int, length: int, vocab: int, seed: int = 1041) -> torch.Tensor:
    """Prompt tokens drawn uniformly from the vocabulary (PCG64 ``default_rng(seed)``)."""
    return torch.from_numpy(np.random.default_rng(seed).integers(0, vocab, (batch, length)).astype(np.int64))
