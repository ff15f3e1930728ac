"""Weight-only int8 (W8A16) for the decoder's linear layers, by module
replacement.

Interface: the reference's quantisation stage (src/quantization/int8.py:32-100)
-- the ``QuantizedLinearInt8`` module (buffers ``weight_q``, ``scale``,
``bias``; ``from_linear``, ``dequantized_weight``, ``num_bytes``) and
``quantize_model_int8(model)`` returning ``layers_quantized`` /
``bytes_before`` / ``bytes_after``.

What the modules hold and run here:

* ``weight_q`` -- the int8 codes, [out_features, in_features], in nn.Linear's
  own row order, so the HIP kernels stream them as they are (no repacking);
* ``scale`` -- one fp32 step per output feature; an output feature's weights
  are ``weight_q[j] * scale[j]``;
* ``bias`` -- the original bias (its own dtype) or None.

Quantisation (``quantize_int8_weight``: one wave per weight row, on the GPU)
and the product (``w8a16_linear``: int8 codes widened in registers, fp32
accumulation, the scale applied per output feature in the epilogue) are both
gfx950 HIP kernels; nothing falls back to torch or the CPU, so a model must
be on the GPU to be quantised or run.  Only the linears inside
``model.model.layers`` are replaced (attention q/k/v/o and the MLP's
gate/up/down); the embedding and ``lm_head`` keep their dtype.  The modules
are ordinary callables, so HF's forward, ``patch_model_with_fused_kernels``
(whose FusedMLP then runs the int8 gate/up kernel) and the graph-captured
decoder all use them unchanged.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from ..kernels.w8a16_matmul_hip import quantize_int8_weight, w8a16_linear

__all__ = ["QuantizedLinearInt8", "quantize_model_int8"]


def _nbytes(*tensors: Optional[torch.Tensor]) -> int:
    return sum(t.numel() * t.element_size() for t in tensors if t is not None)


class QuantizedLinearInt8(nn.Module):
    """An ``nn.Linear`` stand-in whose weight is stored as int8 codes plus one
    fp32 scale per output feature: ``y = x @ (weight_q * scale[:, None]).T +
    bias``, computed by the W8A16 kernel without ever forming the 16-bit
    weight.  It has no parameters (inference only); codes, scales and bias
    are buffers, so ``.to()``, ``state_dict`` and graph capture see them."""

    def __init__(self, weight_q: torch.Tensor, scale: torch.Tensor, bias: Optional[torch.Tensor]):
        super().__init__()
        if weight_q.dtype != torch.int8 or weight_q.dim() != 2:
            raise ValueError(f"weight_q must be a 2-D int8 tensor, got {weight_q.dtype} {tuple(weight_q.shape)}")
        if scale.shape != weight_q.shape[:1]:
            raise ValueError(f"scale must hold one value per output feature ({weight_q.shape[0]}), "
                             f"got {tuple(scale.shape)}")
        self.out_features, self.in_features = weight_q.shape
        self.register_buffer("weight_q", weight_q)
        self.register_buffer("scale", scale)
        self.register_buffer("bias", bias)

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "QuantizedLinearInt8":
        """Quantises ``linear`` on its GPU: per output feature, scale =
        max(max|w| / 127, 1e-8) and codes = clamp(round-half-even(w / scale),
        -127, 127).  The bias is copied, not shared."""
        codes, scale = quantize_int8_weight(linear.weight)
        bias = None if linear.bias is None else linear.bias.detach().clone()
        return cls(codes, scale, bias)

    def dequantized_weight(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """The dense [out_features, in_features] weight the codes stand for,
        in ``dtype`` (for checks and comparisons; the forward never builds
        it)."""
        dense = self.weight_q.to(torch.float32) * self.scale.to(torch.float32).unsqueeze(1)
        return dense.to(dtype)

    def num_bytes(self) -> int:
        """Bytes of device memory the module holds: codes, scales and bias."""
        return _nbytes(self.weight_q, self.scale, self.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return w8a16_linear(x, self.weight_q, self.scale, self.bias)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}"


def quantize_model_int8(model: nn.Module) -> dict:
    """Replaces, in place, every ``nn.Linear`` under ``model.model.layers``
    with a ``QuantizedLinearInt8`` and reports how many were replaced and the
    bytes of those layers before and after (weights, scales, biases).  A
    model whose decoder layers hold no ``nn.Linear`` is left as it is and
    reports 0 replacements, so callers should check the count."""
    decoder_layers = model.model.layers
    # (parent, attribute) of every linear, listed before the first swap so the
    # walk never visits a replacement; each 16-bit linear is released as soon
    # as its replacement is in place.
    slots = [(parent, name) for parent in decoder_layers.modules()
             for name, child in parent.named_children() if isinstance(child, nn.Linear)]
    bytes_16bit = bytes_int8 = 0
    for parent, name in slots:
        linear = getattr(parent, name)
        quantized = QuantizedLinearInt8.from_linear(linear)
        bytes_16bit += _nbytes(linear.weight, linear.bias)
        bytes_int8 += quantized.num_bytes()
        setattr(parent, name, quantized)
        del linear
    if torch.cuda.is_available():
        torch.cuda.empty_cache()  # hand the released 16-bit weights back to the device
    return {"layers_quantized": len(slots), "bytes_before": bytes_16bit, "bytes_after": bytes_int8}
