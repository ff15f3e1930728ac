"""Module replacement that swaps the MI355X fused kernels into Qwen2-style
decoder layers: drop-in for the reference's
``src/engine/fused_norm_activation_patch.py``.

Same surface and behaviour as the reference (:29-99):

* RMSNorm children are matched by class name in ``RMSNORM_CLASS_NAMES`` plus
  the ``weight`` and ``variance_epsilon`` attributes and replaced by
  ``FusedRMSNorm``; MLP children are matched by class name in
  ``MLP_CLASS_NAMES`` plus ``gate_proj``/``up_proj``/``down_proj`` and
  replaced by ``FusedMLP``.
* Replacement is ``setattr`` on the parent (the module registry is updated);
  no ``forward`` is rebound on an existing instance.
* The replacements reuse the original ``nn.Parameter`` / ``nn.Linear``
  objects, so weights are shared, not copied, and other module surgery
  (e.g. quantised Linear layers) composes with ``FusedMLP``.
* ``patch_model_with_fused_kernels`` returns ``{"rmsnorm": n, "mlp": n}``; an
  unrecognised architecture silently replaces nothing, so callers check
  the counts.

Beyond the reference: ``fuse_residual=True`` (off by default, so the default
behaviour and return value are the reference's) also replaces each decoder
layer by ``FusedDecoderLayer``, which runs the post-attention residual add
inside the post-attention RMSNorm (``fused_add_rmsnorm``) -- the "fused
RMSNorm + residual" the reference plans (docs/architecture-cuda.md:94).  The
result is bit-identical to the unfused layer with the fused kernels; the
count appears as ``"add_rmsnorm"``.  ``fuse_gate_up=True`` (also off by
default) lets each FusedMLP run its gate / up projections and the
SiLU-and-mul in one kernel (``fused_gate_up_silu``: weight streaming for
decode batches, a tiled MFMA GEMM for prefill); the projections are then not
rounded before the activation, which changes results by that rounding.  The
count appears as ``"gate_up"``.  ``hip_down=True`` (off by default) runs each
FusedMLP's down projection on the HIP 16-bit linear (``linear16``: weight
streaming on MFMA) for inputs of at most ``LINEAR16_MAX_ROWS`` rows, where
torch's linear is far from HBM bandwidth; its fp32 sums run in another order
than hipBLASLt's, so outputs may differ in the last bit.  The count appears as
``"down"``.
"""
from __future__ import annotations

import torch

from ..kernels.fused_rmsnorm_hip import fused_add_rmsnorm, fused_rmsnorm
from ..kernels.fused_gate_up_hip import fused_gate_up_silu
from ..kernels.fused_swiglu_hip import fused_silu_mul
from ..kernels.linear16_hip import LINEAR16_MAX_ROWS, linear16
from ..kernels.w8a16_matmul_hip import fused_gate_up_silu_w8a16
from ..quantization.int8 import QuantizedLinearInt8

__all__ = ["RMSNORM_CLASS_NAMES", "MLP_CLASS_NAMES", "DECODER_LAYER_CLASS_NAMES", "FusedRMSNorm", "FusedMLP",
           "FusedDecoderLayer", "patch_model_with_fused_kernels"]

RMSNORM_CLASS_NAMES = {"Qwen2RMSNorm", "LlamaRMSNorm", "MistralRMSNorm", "RMSNorm"}
MLP_CLASS_NAMES = {"Qwen2MLP", "LlamaMLP", "MistralMLP"}
DECODER_LAYER_CLASS_NAMES = {"Qwen2DecoderLayer", "LlamaDecoderLayer", "MistralDecoderLayer"}
_DECODER_LAYER_PARTS = ("self_attn", "mlp", "input_layernorm", "post_attention_layernorm")


class FusedRMSNorm(torch.nn.Module):
    """Wraps an existing RMSNorm module's weight and eps; forward runs the
    fused HIP kernel.  Holds the original ``nn.Parameter`` object itself."""

    def __init__(self, orig_module: torch.nn.Module):
        super().__init__()
        self.weight = orig_module.weight
        self.variance_epsilon = orig_module.variance_epsilon

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return fused_rmsnorm(hidden_states, self.weight, self.variance_epsilon)


def _plain_linear(m: torch.nn.Module) -> bool:
    return type(m) is torch.nn.Linear and m.bias is None


class FusedMLP(torch.nn.Module):
    """Wraps an existing SwiGLU MLP's three projections and replaces the
    ``act_fn(gate) * up`` step with the fused SiLU-and-mul kernel.  SiLU is
    fixed, as in the reference; the projection modules are reused.

    With ``fuse_gate_up=True``, fp16 / bf16 inputs whose projections are
    plain bias-free ``nn.Linear`` layers of x's dtype with k a multiple of 8
    take ``fused_gate_up_silu`` instead (decode steps and prefill alike), and
    those whose projections are bias-free ``QuantizedLinearInt8`` layers take
    ``fused_gate_up_silu_w8a16``: gate, up and the activation in one kernel.
    The projection kind is checked at each call, so a model quantised after
    patching switches to the int8 kernel.  Other inputs take the reference
    path.

    With ``hip_down=True``, a down projection that is a plain ``nn.Linear``
    of the activation's dtype (fp16 / bf16) runs on ``linear16`` for inputs
    of at most ``LINEAR16_MAX_ROWS`` rows (decode steps); larger inputs, and
    other projection kinds, call the module."""

    def __init__(self, orig_module: torch.nn.Module, fuse_gate_up: bool = False, hip_down: bool = False):
        super().__init__()
        self.gate_proj = orig_module.gate_proj
        self.up_proj = orig_module.up_proj
        self.down_proj = orig_module.down_proj
        self.fuse_gate_up = bool(fuse_gate_up) and self.gate_up_fusable()
        self.hip_down = bool(hip_down) and self.down_hip_capable()

    def gate_up_kind(self) -> str | None:
        """Which fused gate/up kernel can read the projections: ``"16bit"``
        (plain bias-free Linear layers of one shape with k a multiple of 8),
        ``"int8"`` (bias-free QuantizedLinearInt8 layers of one shape and
        scale dtype) or None."""
        g, u = self.gate_proj, self.up_proj
        if (_plain_linear(g) and _plain_linear(u) and g.weight.shape == u.weight.shape
                and g.weight.shape[1] % 8 == 0):
            return "16bit"
        if (type(g) is QuantizedLinearInt8 and type(u) is QuantizedLinearInt8 and g.bias is None and u.bias is None
                and g.weight_q.shape == u.weight_q.shape and g.scale.dtype == u.scale.dtype):
            return "int8"
        return None

    def gate_up_fusable(self) -> bool:
        return self.gate_up_kind() is not None

    def down_hip_capable(self) -> bool:
        """Whether ``linear16`` can run the down projection: a plain
        ``nn.Linear`` (bias allowed)."""
        return type(self.down_proj) is torch.nn.Linear

    def down(self, activated: torch.Tensor) -> torch.Tensor:
        """The down projection: ``linear16`` for decode-sized 16-bit inputs
        when ``hip_down`` is on, else the module itself."""
        d = self.down_proj
        if (self.hip_down and type(d) is torch.nn.Linear and activated.dtype == d.weight.dtype
                and activated.dtype in (torch.float16, torch.bfloat16)
                and activated.numel() <= LINEAR16_MAX_ROWS * activated.shape[-1]):
            return linear16(activated, d.weight, d.bias)
        return d(activated)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.fuse_gate_up and x.dtype in (torch.float16, torch.bfloat16):
            kind = self.gate_up_kind()
            g, u = self.gate_proj, self.up_proj
            if kind == "16bit" and x.dtype == g.weight.dtype == u.weight.dtype:
                return self.down(fused_gate_up_silu(x, g.weight, u.weight))
            if kind == "int8":
                return self.down(fused_gate_up_silu_w8a16(x, g.weight_q, g.scale, u.weight_q, u.scale))
        gate = self.gate_proj(x)
        up = self.up_proj(x)
        activated = fused_silu_mul(gate, up)
        return self.down(activated)


class FusedDecoderLayer(torch.nn.Module):
    """A pre-norm decoder layer (Qwen2 / Llama / Mistral layout) whose
    post-attention residual add runs inside the post-attention RMSNorm.

    Reuses the layer's own ``self_attn``, ``mlp``, ``input_layernorm`` and
    ``post_attention_layernorm`` modules (already replaced by the fused ones
    if the model was patched) and follows HF's decoder-layer forward:
    input norm -> attention -> residual add + post-attention norm (one fused
    kernel here) -> MLP -> residual add."""

    def __init__(self, orig_layer: torch.nn.Module):
        super().__init__()
        for name in _DECODER_LAYER_PARTS:
            setattr(self, name, getattr(orig_layer, name))
        # plain attributes callers may read from a layer (e.g. attention_type)
        for key, val in vars(orig_layer).items():
            if not key.startswith("_") and not isinstance(val, torch.nn.Module) and not hasattr(self, key):
                setattr(self, key, val)

    def forward(self, hidden_states: torch.Tensor, attention_mask=None, position_ids=None, past_key_values=None,
                use_cache=False, position_embeddings=None, **kwargs) -> torch.Tensor:
        residual = hidden_states
        hidden_states = self.input_layernorm(hidden_states)
        hidden_states, _ = self.self_attn(
            hidden_states=hidden_states,
            attention_mask=attention_mask,
            position_ids=position_ids,
            past_key_values=past_key_values,
            use_cache=use_cache,
            position_embeddings=position_embeddings,
            **kwargs,
        )
        norm = self.post_attention_layernorm
        hidden_states, residual = fused_add_rmsnorm(hidden_states, residual, norm.weight, norm.variance_epsilon)
        hidden_states = self.mlp(hidden_states)
        return residual + hidden_states


def patch_model_with_fused_kernels(model: torch.nn.Module, patch_norm: bool = True,
                                   patch_mlp: bool = True, fuse_residual: bool = False,
                                   fuse_gate_up: bool = False, hip_down: bool = False) -> dict:
    """Replace matching RMSNorm and/or MLP child modules in place (setattr on
    the parent).  Returns ``{"rmsnorm": count, "mlp": count}``.
    ``patch_norm`` / ``patch_mlp`` enable each kernel independently.
    ``fuse_residual`` additionally replaces matching decoder layers by
    ``FusedDecoderLayer`` and adds ``"add_rmsnorm": count`` to the result.
    ``fuse_gate_up`` builds each FusedMLP with ``fuse_gate_up=True`` and adds
    ``"gate_up": count`` (the MLPs whose projections the fused kernel can
    read).  ``hip_down`` builds each FusedMLP with ``hip_down=True`` and adds
    ``"down": count`` (the MLPs whose down projection ``linear16`` can run)."""
    counts = {"rmsnorm": 0, "mlp": 0}
    if fuse_gate_up:
        counts["gate_up"] = 0
    if hip_down:
        counts["down"] = 0
    for parent in list(model.modules()):
        for child_name, child in list(parent.named_children()):
            cls_name = child.__class__.__name__
            if (patch_norm and cls_name in RMSNORM_CLASS_NAMES and hasattr(child, "weight")
                    and hasattr(child, "variance_epsilon")):
                setattr(parent, child_name, FusedRMSNorm(child))
                counts["rmsnorm"] += 1
            elif patch_mlp and cls_name in MLP_CLASS_NAMES and all(
                    hasattr(child, attr) for attr in ("gate_proj", "up_proj", "down_proj")):
                fused = FusedMLP(child, fuse_gate_up=fuse_gate_up, hip_down=hip_down)
                setattr(parent, child_name, fused)
                counts["mlp"] += 1
                if fused.fuse_gate_up:
                    counts["gate_up"] += 1
                if fused.hip_down:
                    counts["down"] += 1
    if fuse_residual:
        counts["add_rmsnorm"] = 0
        for parent in list(model.modules()):
            for child_name, child in list(parent.named_children()):
                if child.__class__.__name__ in DECODER_LAYER_CLASS_NAMES and all(
                        hasattr(child, part) for part in _DECODER_LAYER_PARTS):
                    setattr(parent, child_name, FusedDecoderLayer(child))
                    counts["add_rmsnorm"] += 1
    return counts
