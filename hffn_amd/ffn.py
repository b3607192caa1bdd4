"""Isolated HFFN FFN on the HIP runtime: the layer constructor of the FFN leaf
(``runtime/gpu/nvidia/ffn/inference/hffn_ffn_cuda/layers.py:9-14``)."""
from __future__ import annotations

import torch

from .runtime import HFFNLayer
from .synth import CompactLayer


def hip_layer(layer: CompactLayer, device: str | torch.device | None = None) -> HFFNLayer:
    """``HFFNLayer`` of a compact hidden-major layer (numpy arrays); the output-major store is built on the device.
    A ``bf16`` layer is stored with bfloat16 values (its float32 values are exactly representable)."""
    t = torch.from_numpy
    dtype = torch.bfloat16 if layer.value_dtype == "bf16" else torch.float32
    return HFFNLayer.from_hidden_major(layer.d_model, layer.d_ff, t(layer.b_up), t(layer.up_offsets), t(layer.up_idx),
                                       t(layer.up_val).to(dtype), t(layer.b_down), t(layer.down_offsets),
                                       t(layer.down_idx), t(layer.down_val).to(dtype), device=device)


cuda_layer = hip_layer  # the reference name (the device is "cuda" to PyTorch-ROCm)
