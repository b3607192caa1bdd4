"""Pythia (GPT-NeoX) whose FFNs run dense or on the HFFN HIP runtime: the compact export format, the two-arm
loader and its hook, and writers of random-init Pythia-shaped checkpoints with synthetic exports.

Interfaces kept from the reference (paths relative to its root):

* the export format ``hffn_training_compact_g4_v2`` (``runtime/common/pythia/hffn_pythia/export.py:13-57``): one
  ``torch.save`` dict per layer, hidden-major ``up_*``/``down_*`` arrays, biases, and the four-group hidden
  partition; ``read_layer(path, groups=False)`` returns its arrays and raises ``ValueError`` on a malformed file;
* ``load_pythia(model_dir, export_dir, ffn, device, make_runtime)`` - both the NVIDIA leaf's loader
  (``runtime/gpu/nvidia/llm/inference/hffn_pythia_cuda/model.py:23-28``, which builds the GPU runtime) and the shared
  one (``runtime/common/pythia/hffn_pythia/model.py:82-111``, which takes ``make_runtime``); the HFFN arm exposes
  ``model.hffn_runtime``;
* ``HFFNMLP(runtime, index)`` (``model.py:27-37``) in place of ``block.mlp``; ``layer_from_export`` (leaf
  ``model.py:11-15``); ``share_non_ffn(model, source)`` (``model.py:114-124``).

How this module builds the arms:

* every model is built from its ``config.json``; the HFFN arm is built with a zero-width MLP (``intermediate_size``
  set to 0 while the modules are created, so the two projections hold no weight) and each block's MLP is then
  replaced by ``HFFNMLP``: no dense FFN tensor is ever created for that arm;
* the non-FFN tensors come from ``model.safetensors`` through ``load_state_dict(strict=False)``; the only keys allowed
  to differ are the FFN's own and the attention buffers that older checkpoints carry and the model rebuilds itself;
* the dense arm's two projections are the export's hidden-major stores read as CSR matrices (``up``: rows are
  neurons over the input features; ``down``: rows are neurons over the outputs, transposed), densified by torch.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
from torch import nn

FORMAT = "hffn_training_compact_g4_v2"
# The arrays of one export and their dtypes (export.py:13-17): hidden-major offsets over d_ff + 1 entries, int16
# feature indices, float32 values and biases.
ARRAYS = {
    "up_row_offsets": torch.int32, "up_idx": torch.int16, "up_val": torch.float32, "b_up": torch.float32,
    "down_row_offsets": torch.int32, "down_idx": torch.int16, "down_val": torch.float32, "b_down": torch.float32,
}
GROUPS = "group_hidden_offsets"  # int32[5]: the four hidden groups of the CPU runtimes, from 0 to d_ff
# Attention buffers that checkpoints of older transformers releases hold and current GPT-NeoX modules recompute.
REBUILT_BUFFERS = ("attention.bias", "attention.masked_bias", "attention.rotary_emb.inv_freq")


# ------------------------------------------------------------------------------------------------- export format

def _is_partition(bounds: torch.Tensor, total: int) -> bool:
    """Whether ``bounds`` runs from 0 to ``total`` without ever decreasing."""
    return bounds.numel() >= 1 and int(bounds[0]) == 0 and int(bounds[-1]) == total and not bool((bounds[1:] < bounds[:-1]).any())


def read_layer(path: str | Path, *, groups: bool = False) -> dict:
    """One export file as a dict of contiguous CPU tensors plus ``d_model`` and ``d_ff``; with ``groups`` also
    ``group_hidden_offsets``. A file that is not a valid ``hffn_training_compact_g4_v2`` layer raises ``ValueError``
    naming the first problem found."""
    path = Path(path)
    blob = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(blob, dict) or blob.get("format") != FORMAT:
        raise ValueError(f"{path}: not a {FORMAT} layer file")
    d_model, d_ff = int(blob["d_model"]), int(blob["d_ff"])
    layer: dict = {"d_model": d_model, "d_ff": d_ff}
    wanted = dict(ARRAYS, **({GROUPS: torch.int32} if groups else {}))
    for name, dtype in wanted.items():
        array = blob.get(name)
        if not isinstance(array, torch.Tensor) or array.dtype != dtype or array.dim() != 1:
            raise ValueError(f"{path}: {name} is missing or not a 1-D {dtype} array")
        layer[name] = array.contiguous()
    problems = []
    if layer["b_up"].numel() != d_ff:
        problems.append(f"b_up has {layer['b_up'].numel()} entries for d_ff {d_ff}")
    if layer["b_down"].numel() != d_model:
        problems.append(f"b_down has {layer['b_down'].numel()} entries for d_model {d_model}")
    for side in ("up", "down"):
        offsets, index, values = layer[f"{side}_row_offsets"], layer[f"{side}_idx"], layer[f"{side}_val"]
        if index.numel() != values.numel():
            problems.append(f"{side}: {index.numel()} indices for {values.numel()} values")
        elif offsets.numel() != d_ff + 1 or not _is_partition(offsets, values.numel()):
            problems.append(f"{side}: the row offsets do not split the {values.numel()} slots over {d_ff} neurons")
        elif index.numel() and not (0 <= int(index.min()) and int(index.max()) < d_model):
            problems.append(f"{side}: feature index outside [0, {d_model})")
    if groups and (layer[GROUPS].numel() != 5 or not _is_partition(layer[GROUPS], d_ff)):
        problems.append(f"{GROUPS} is not a partition of the {d_ff} neurons into four groups")
    if problems:
        raise ValueError(f"{path}: " + "; ".join(problems))
    return layer


def layer_path(export_dir: str | Path, index: int) -> Path:
    """Where layer ``index`` of an export lives: ``<export_dir>/layer<index>/<FORMAT>.pt``."""
    return Path(export_dir) / f"layer{index}" / f"{FORMAT}.pt"


def read_layers(export_dir: str | Path, count: int) -> list[dict]:
    return [read_layer(layer_path(export_dir, index)) for index in range(count)]


def write_layer(path: str | Path, layer: dict) -> None:
    """Save one layer dict (the keys ``read_layer`` returns) in the export format."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    d_ff = int(layer["d_ff"])
    blob = {"format": FORMAT, "d_model": int(layer["d_model"]), "d_ff": d_ff}
    blob.update({name: torch.as_tensor(layer[name]).to(dtype).contiguous() for name, dtype in ARRAYS.items()})
    quarters = torch.tensor([d_ff * g // 4 for g in range(5)], dtype=torch.int32)
    blob[GROUPS] = torch.as_tensor(layer.get(GROUPS, quarters)).to(torch.int32).contiguous()
    torch.save(blob, path)


def hidden_of_slot(layer: dict, side: str) -> torch.Tensor:
    """Owner neuron of every slot of one side, int64[nnz] (neuron r repeated for each of its slots)."""
    counts = (layer[f"{side}_row_offsets"][1:] - layer[f"{side}_row_offsets"][:-1]).long()
    return torch.arange(layer["d_ff"]).repeat_interleave(counts)


def export_of_compact(compact) -> dict:
    """The layer dict of a compact hidden-major layer (``hffn_amd.synth.CompactLayer``)."""
    pairs = (("up_row_offsets", "up_offsets"), ("up_idx", "up_idx"), ("up_val", "up_val"), ("b_up", "b_up"),
             ("down_row_offsets", "down_offsets"), ("down_idx", "down_idx"), ("down_val", "down_val"),
             ("b_down", "b_down"), (GROUPS, "groups"))
    layer = {key: torch.from_numpy(np.ascontiguousarray(getattr(compact, field))) for key, field in pairs}
    layer.update(d_model=compact.d_model, d_ff=compact.d_ff)
    return layer


def dense_projections(layer: dict) -> tuple[torch.Tensor, torch.Tensor]:
    """float32 ``W_up [d_ff, d_model]`` and ``W_down [d_model, d_ff]``, zero outside the support: each side's
    hidden-major store read as a CSR matrix with one row per neuron."""
    shape = (layer["d_ff"], layer["d_model"])

    def csr(side: str) -> torch.Tensor:
        return torch.sparse_csr_tensor(layer[f"{side}_row_offsets"].long(), layer[f"{side}_idx"].long(),
                                       layer[f"{side}_val"].float(), size=shape).to_dense()

    return csr("up"), csr("down").T.contiguous()


# ----------------------------------------------------------------------------------------------------- the hook

class HFFNMLP(nn.Module):
    """``block.mlp`` of the HFFN arm: the block's FFN input, flattened to tokens, through layer ``index`` of the
    runtime. The result is a view of the runtime's output buffer; the block adds it into its residual before the next
    FFN call overwrites it."""

    def __init__(self, runtime, index: int) -> None:
        super().__init__()
        self.runtime, self.index = runtime, index

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        width = hidden_states.shape[-1]
        return self.runtime.forward(self.index, hidden_states.reshape(-1, width)).view(hidden_states.shape)


def layer_from_export(layer: dict, device: str | torch.device | None = None):
    """``HFFNLayer`` of one layer dict; its output-major down store is built on the device."""
    from .runtime import HFFNLayer
    return HFFNLayer.from_hidden_major(layer["d_model"], layer["d_ff"], layer["b_up"], layer["up_row_offsets"],
                                       layer["up_idx"], layer["up_val"], layer["b_down"], layer["down_row_offsets"],
                                       layer["down_idx"], layer["down_val"], device=device)


def hip_runtime(layers: list[dict], device: str | torch.device = "cuda"):
    """The leaf's runtime of an export (the reference leaf's ``_runtime``, ``hffn_pythia_cuda/model.py:18-20``): a
    ``PreparedRuntime``, whose decode calls launch from per-(layer, N) plans."""
    from .prepared_runtime import PreparedRuntime
    return PreparedRuntime([layer_from_export(layer, device) for layer in layers], device)


# --------------------------------------------------------------------------------------------------- the loader

def _build(config, ffn_width: int | None = None) -> nn.Module:
    """A float32 causal LM of ``config``; with ``ffn_width`` the MLPs are created that wide (0: no FFN weights) and
    the config keeps its own width afterwards."""
    from transformers import AutoModelForCausalLM
    if ffn_width is None:
        return AutoModelForCausalLM.from_config(config, dtype=torch.float32)
    width = config.intermediate_size
    config.intermediate_size = ffn_width
    try:
        model = AutoModelForCausalLM.from_config(config, dtype=torch.float32)
    finally:
        config.intermediate_size = width
    model.config.intermediate_size = width
    return model


def _is_ffn(name: str) -> bool:
    return ".mlp." in name


def _load_attention_and_embeddings(model: nn.Module, checkpoint: Path) -> None:
    """Every non-FFN tensor of the model from ``checkpoint`` (safetensors). FFN keys are ignored on both sides; the
    checkpoint may also hold buffers the model rebuilds (``REBUILT_BUFFERS``); anything else that does not match is a
    ``ValueError``."""
    from safetensors.torch import load_file
    state = {name: tensor for name, tensor in load_file(str(checkpoint)).items() if not _is_ffn(name)}
    missing, unexpected = model.load_state_dict(state, strict=False)
    missing = [name for name in missing if not _is_ffn(name)]
    unexpected = [name for name in unexpected if not name.endswith(REBUILT_BUFFERS)]
    if missing or unexpected:
        raise ValueError(f"{checkpoint} does not fit the model: missing {sorted(missing)}, extra {sorted(unexpected)}")


def load_pythia(model_dir: str | Path, export_dir: str | Path, ffn: str, device: str | torch.device = "cuda",
                make_runtime=None) -> nn.Module:
    """A Pythia model in eval mode (float32, on ``device``, no gradients) whose FFNs come from ``export_dir``:
    ``ffn="dense"`` runs them as the model's own ``GPTNeoXMLP`` on the densified support, ``ffn="hffn"`` through
    ``HFFNMLP`` and the runtime ``make_runtime(layers)`` builds from the layer dicts (default: ``hip_runtime`` on
    ``device``), which is exposed as ``model.hffn_runtime`` (None for the dense arm)."""
    from transformers import AutoConfig
    if ffn not in ("dense", "hffn"):
        raise ValueError(f"ffn is 'dense' or 'hffn', not {ffn!r}")
    model_dir = Path(model_dir)
    config = AutoConfig.from_pretrained(str(model_dir))
    model = _build(config, ffn_width=0 if ffn == "hffn" else None)
    _load_attention_and_embeddings(model, model_dir / "model.safetensors")
    blocks = model.gpt_neox.layers
    layers = read_layers(export_dir, len(blocks))
    runtime = None
    if ffn == "dense":
        with torch.no_grad():
            for block, layer in zip(blocks, layers):
                up, down = block.mlp.dense_h_to_4h, block.mlp.dense_4h_to_h
                if tuple(up.weight.shape) != (layer["d_ff"], layer["d_model"]):
                    raise ValueError(f"export layer of {layer['d_model']} x {layer['d_ff']} does not fit an MLP of "
                                     f"{tuple(up.weight.shape[::-1])}")
                w_up, w_down = dense_projections(layer)
                up.weight.copy_(w_up)
                up.bias.copy_(layer["b_up"])
                down.weight.copy_(w_down)
                down.bias.copy_(layer["b_down"])
    else:
        runtime = make_runtime(layers) if make_runtime is not None else hip_runtime(layers, device)
        for index, block in enumerate(blocks):
            block.mlp = HFFNMLP(runtime, index)
        if any(_is_ffn(name) for name, _ in model.named_parameters()):
            raise RuntimeError("the HFFN arm still holds FFN parameters")
    model = model.to(device).eval().requires_grad_(False)
    model.hffn_runtime = runtime
    return model


@torch.no_grad()
def share_non_ffn(model: nn.Module, source: nn.Module) -> None:
    """Point every non-FFN parameter of ``model`` at the tensor ``source`` holds under the same name (both arms loaded
    from one checkpoint), so that two arms in one process read one copy of those weights and differ by their FFNs
    only."""
    for name, parameter in source.named_parameters():
        if _is_ffn(name):
            continue
        owner_name, _, attribute = name.rpartition(".")
        owner = model.get_submodule(owner_name)
        current = getattr(owner, attribute)
        if current.shape != parameter.shape:
            raise ValueError(f"{name}: {tuple(current.shape)} in the model, {tuple(parameter.shape)} in the source")
        setattr(owner, attribute, parameter)


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
    """Write ``config.json`` and a ``model.safetensors`` of the non-FFN tensors of a model initialised by its classes
    after ``torch.manual_seed(seed)``. Returns the config."""
    from safetensors.torch import save_file
    config = pythia_config(**config_overrides)
    model_dir = Path(model_dir)
    model_dir.mkdir(parents=True, exist_ok=True)
    config.save_pretrained(str(model_dir))
    torch.manual_seed(seed)
    model = _build(config, ffn_width=0)
    save_file({name: tensor.contiguous() for name, tensor in model.state_dict().items() if not _is_ffn(name)},
              str(model_dir / "model.safetensors"))
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


def synthetic_prompts(batch: int, length: int, vocab: int, seed: int = 1041) -> torch.Tensor:
    """Prompt tokens drawn uniformly from the vocabulary (PCG64 ``default_rng(seed)``)."""
    return torch.from_numpy(np.random.default_rng(seed).integers(0, vocab, (batch, length)).astype(np.int64))
