"""HIP segment-LoRA kernels (export surface of multi_lora/kernels/__init__.py:3-7)."""

from .lora_ops import (
    Workspace,
    sgemm_lora_a_fwd,
    sgemm_lora_a_multi_fwd,
    sgemm_lora_b_fwd,
    sgemm_lora_b_multi_fwd,
)
from .rmsnorm import fuse_rmsnorm, fused_add_rmsnorm, rmsnorm_fwd
from .scatter_bank import scatter_stage

__all__ = [
    "Workspace",
    "sgemm_lora_a_fwd",
    "sgemm_lora_b_fwd",
    "scatter_stage",
    "sgemm_lora_a_multi_fwd",
    "sgemm_lora_b_multi_fwd",
    "rmsnorm_fwd",
    "fuse_rmsnorm",
    "fused_add_rmsnorm",
]
