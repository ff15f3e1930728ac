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
"""
from __future__ import annotations

import torch

from ..kernels.fused_rmsnorm_hip import fused_rmsnorm
from ..kernels.fused_swiglu_hip import fused_silu_mul

__all__ = ["RMSNORM_CLASS_NAMES", "MLP_CLASS_NAMES", "FusedRMSNorm", "FusedMLP",
           "patch_model_with_fused_kernels"]

RMSNORM_CLASS_NAMES = {"Qwen2RMSNorm", "LlamaRMSNorm", "MistralRMSNorm", "RMSNorm"}
MLP_CLASS_NAMES = {"Qwen2MLP", "LlamaMLP", "MistralMLP"}


class FusedRMSNorm(torch.nn.Module):
    """Wraps an existing RMSNorm module's weight and eps; forward runs the
    fused HIP kernel.  Holds the original ``nn.Parameter`` object itself."""

    def __init__(self, orig_module: torch.nn.Module):
        super().__init__()
        self.weight = orig_module.weight
        self.variance_epsilon = orig_module.variance_epsilon

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return fused_rmsnorm(hidden_states, self.weight, self.variance_epsilon)


class FusedMLP(torch.nn.Module):
    """Wraps an existing SwiGLU MLP's three projections and replaces the
    ``act_fn(gate) * up`` step with the fused SiLU-and-mul kernel.  SiLU is
    fixed, as in the reference; the projection modules are reused."""

    def __init__(self, orig_module: torch.nn.Module):
        super().__init__()
        self.gate_proj = orig_module.gate_proj
        self.up_proj = orig_module.up_proj
        self.down_proj = orig_module.down_proj

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate = self.gate_proj(x)
        up = self.up_proj(x)
        activated = fused_silu_mul(gate, up)
        return self.down_proj(activated)


def patch_model_with_fused_kernels(model: torch.nn.Module, patch_norm: bool = True,
                                   patch_mlp: bool = True) -> dict:
    """Replace matching RMSNorm and/or MLP child modules in place (setattr on
    the parent).  Returns ``{"rmsnorm": count, "mlp": count}``.
    ``patch_norm`` / ``patch_mlp`` enable each kernel independently."""
    counts = {"rmsnorm": 0, "mlp": 0}
    for parent in list(model.modules()):
        for child_name, child in list(parent.named_children()):
            cls_name = child.__class__.__name__
            if (patch_norm and cls_name in RMSNORM_CLASS_NAMES and hasattr(child, "weight")
                    and hasattr(child, "variance_epsilon")):
                setattr(parent, child_name, FusedRMSNorm(child))
                counts["rmsnorm"] += 1
            elif patch_mlp and cls_name in MLP_CLASS_NAMES and all(
                    hasattr(child, attr) for attr in ("gate_proj", "up_proj", "down_proj")):
                setattr(parent, child_name, FusedMLP(child))
                counts["mlp"] += 1
    return counts
