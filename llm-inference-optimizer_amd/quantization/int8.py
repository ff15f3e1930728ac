"""INT8 weight-only quantisation of a loaded model, by module replacement.

Mirrors the reference's quantisation stage (src/quantization/int8.py): every
``nn.Linear`` inside ``model.model.layers`` (q/k/v/o and gate/up/down) is
replaced in its parent's registry by a ``QuantizedLinearInt8`` holding int8
weights and one fp32 scale per output feature; embeddings and ``lm_head``
keep their dtype (for Qwen2.5-1.5B they are tied).  The replacement modules
are plain callables, so HF's forward and the graph-captured decoder use them
unchanged, and they compose with ``patch_model_with_fused_kernels`` (FusedMLP
calls its projections as modules).

Both the quantiser and the forward run as gfx950 HIP kernels
(``quantize_int8_weight`` and ``w8a16_linear``); there is no torch or CPU
fallback, so the model must be on the GPU.
"""
from __future__ import annotations

import gc
from typing import Optional

import torch
import torch.nn as nn

from ..kernels.w8a16_matmul_hip import quantize_int8_weight, w8a16_linear

__all__ = ["QuantizedLinearInt8", "quantize_model_int8"]


class QuantizedLinearInt8(nn.Module):
    """Drop-in replacement for nn.Linear holding int8 weights plus a
    per-output-channel float32 scale (src/quantization/int8.py:32-63).
    Weights and scales are buffers: an inference-only module."""

    def __init__(self, weight_q: torch.Tensor, scale: torch.Tensor, bias: Optional[torch.Tensor]):
        super().__init__()
        self.register_buffer("weight_q", weight_q)
        self.register_buffer("scale", scale)
        self.register_buffer("bias", bias)  # None is allowed
        self.out_features, self.in_features = weight_q.shape

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "QuantizedLinearInt8":
        """Quantise ``linear`` (on the GPU) with the HIP quantiser: scale =
        max(max|w_row| / 127, 1e-8), w_q = clamp(round(w / scale), -127, 127)."""
        w_q, scale = quantize_int8_weight(linear.weight)
        bias = linear.bias.detach().clone() if linear.bias is not None else None
        return cls(w_q, scale, bias)

    def dequantized_weight(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        return (self.weight_q.float() * self.scale[:, None]).to(dtype)

    def num_bytes(self) -> int:
        total = self.weight_q.numel() * self.weight_q.element_size()
        total += self.scale.numel() * self.scale.element_size()
        if self.bias is not None:
            total += self.bias.numel() * self.bias.element_size()
        return total

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return w8a16_linear(x, self.weight_q, self.scale, self.bias)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}"


def _linear_bytes(linear: nn.Linear) -> int:
    total = linear.weight.numel() * linear.weight.element_size()
    if linear.bias is not None:
        total += linear.bias.numel() * linear.bias.element_size()
    return total


def quantize_model_int8(model: nn.Module) -> dict:
    """Replaces every nn.Linear inside ``model.model.layers`` with a
    QuantizedLinearInt8, in place (src/quantization/int8.py:73-100).  Returns
    ``{"layers_quantized", "bytes_before", "bytes_after"}``; callers should
    check ``layers_quantized > 0`` (an unrecognised layout quantises nothing)."""
    layers_root = model.model.layers
    layers_quantized = 0
    bytes_before = 0
    bytes_after = 0

    for parent in list(layers_root.modules()):
        for child_name, child in list(parent.named_children()):
            if isinstance(child, nn.Linear):
                bytes_before += _linear_bytes(child)
                quantized = QuantizedLinearInt8.from_linear(child)
                bytes_after += quantized.num_bytes()
                setattr(parent, child_name, quantized)
                layers_quantized += 1

    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()

    return {
        "layers_quantized": layers_quantized,
        "bytes_before": bytes_before,
        "bytes_after": bytes_after,
    }
