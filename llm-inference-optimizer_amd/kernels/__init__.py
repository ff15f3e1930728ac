"""MI355X (gfx950) fused kernels behind the reference's launcher API."""
from .fused_rmsnorm_hip import fused_add_rmsnorm, fused_rmsnorm, naive_rmsnorm_reference
from .fused_swiglu_hip import fused_silu_mul, naive_silu_mul_reference

__all__ = ["fused_rmsnorm", "fused_add_rmsnorm", "naive_rmsnorm_reference", "fused_silu_mul", "naive_silu_mul_reference"]
