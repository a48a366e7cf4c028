"""MI355X-native segment-LoRA hot path: shrink, expand (single and
multi-slice) and fused RMSNorm as hand-written gfx950 HIP kernels behind
the host API of multi_lora (backend, segment metadata, slot pool, layers).
"""

from .backend import HipLoRABackend, LoRABackend, get_lora_backend
from .batch_info import (
    BatchLoRAInfo,
    KernelInputMetaData,
    empty_kernel_input_metadata,
    fill_column,
    group_rows,
    segment_lens,
    write_kernel_input_metadata,
)
from .eviction import EvictionPolicy
from .layers import (LinearWithLoRA, QKVProjGroup, fuse_gate_up_projections, fuse_qkv_projections, lora_delta,
                     set_lora_enabled)
from .manager import MultiLoRAManager
from .pool import LoRAMemoryPool
from .weights import AdapterWeights

__all__ = [
    "AdapterWeights",
    "BatchLoRAInfo",
    "EvictionPolicy",
    "HipLoRABackend",
    "KernelInputMetaData",
    "LinearWithLoRA",
    "LoRABackend",
    "LoRAMemoryPool",
    "MultiLoRAManager",
    "QKVProjGroup",
    "empty_kernel_input_metadata",
    "fill_column",
    "fuse_gate_up_projections",
    "fuse_qkv_projections",
    "get_lora_backend",
    "group_rows",
    "lora_delta",
    "segment_lens",
    "set_lora_enabled",
    "write_kernel_input_metadata",
]
