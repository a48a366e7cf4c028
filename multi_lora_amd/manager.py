"""Per-step orchestration: adapters -> slots -> segment table -> wrapped layers.

Reproduces the per-step path of the reference's ``MultiLoRAManager``
(multi_lora/manager.py:172-279) without PEFT: adapters are registered as
``AdapterWeights`` keyed by the dotted names of the model's ``nn.Linear``
modules, and ``convert_to_lora_layers`` wraps those modules in place.
Per step, ``forward_with_lora``

1. merges adjacent rows that use the same adapter (``group_rows``),
2. makes the batch's adapters resident in the slot pool (evicting others),
3. rewrites the resident segment table in place,
4. binds the backend and each module's slot stacks to its wrapper,
5. runs the model.

Environment switches kept from the reference: ``MULTI_LORA_FUSED_QKV``
(default off) and ``MULTI_LORA_FUSED_NORM`` (default on).
"""

from __future__ import annotations

import os
from typing import Dict, Iterable, List, Mapping, Optional

import torch
import torch.nn as nn

from .backend.base import LoRABackend
from .backend.registry import get_lora_backend
from .batch_info import (
    BatchLoRAInfo,
    KernelInputMetaData,
    empty_kernel_input_metadata,
    group_rows,
    write_kernel_input_metadata,
)
from .layers import LinearWithLoRA, fuse_gate_up_projections, fuse_qkv_projections
from .pool import LoRAMemoryPool, LoraName
from .weights import AdapterWeights


def validate_lora_batch(lora_names: List[LoraName], *, max_loras_per_batch: int) -> bool:
    """A batch may use at most ``max_loras_per_batch`` distinct adapters (``None`` counts)."""
    return len(set(lora_names)) <= max_loras_per_batch


class MultiLoRAManager:
    def __init__(
        self,
        model: nn.Module,
        *,
        max_loras_per_batch: int = 4,
        max_lora_rank: int = 64,
        eviction_policy: str = "lru",
        lora_backend: str = "hip",
        lora_target_suffixes: Optional[List[str]] = None,
        device: Optional[torch.device] = None,
        dtype: Optional[torch.dtype] = None,
    ) -> None:
        self.model = model
        self.max_loras_per_batch = max_loras_per_batch
        self.lora_target_suffixes = lora_target_suffixes
        param = next(model.parameters())
        self.pool = LoRAMemoryPool(
            max_loras_per_batch=max_loras_per_batch,
            max_lora_rank=max_lora_rank,
            device=device or param.device,
            dtype=dtype or param.dtype,
            eviction_policy=eviction_policy,
        )
        self._weight_store: Dict[str, AdapterWeights] = {}
        self._lora_backend: LoRABackend = get_lora_backend(lora_backend)
        self.lora_wrappers: Dict[str, LinearWithLoRA] = {}
        self._resident_meta = empty_kernel_input_metadata(device=self.pool.device, dtype=self.pool.dtype)

    @classmethod
    def from_adapters(
        cls, model: nn.Module, adapters: Mapping[str, AdapterWeights], *, convert_lora_layers: bool = True, **kwargs
    ) -> "MultiLoRAManager":
        mgr = cls(model, **kwargs)
        for name, weights in adapters.items():
            mgr.register_adapter(name, weights)
        if convert_lora_layers:
            mgr.convert_to_lora_layers()
        return mgr

    # -- adapters and model surgery ------------------------------------------
    def register_adapter(self, name: str, weights: AdapterWeights) -> None:
        if not name:
            raise ValueError("lora_name cannot be empty")
        if name in self._weight_store:
            raise ValueError(f"LoRA name already registered: {name}")
        weights.validate()
        self._weight_store[name] = weights
        self.pool.ensure_buffers(weights)

    def _target(self, key: str) -> bool:
        if self.lora_target_suffixes is None:
            return True
        return any(key.endswith(sfx) for sfx in self.lora_target_suffixes)

    def convert_to_lora_layers(self) -> None:
        """Wrap every ``nn.Linear`` whose name some adapter targets."""
        keys = set()
        for w in self._weight_store.values():
            keys.update(w.modules.keys())
        keys.update(self.pool.buffers.A.keys())
        for name, module in list(self.model.named_modules()):
            if name in keys and isinstance(module, nn.Linear) and self._target(name):
                parent_name, _, child = name.rpartition(".")
                parent = self.model.get_submodule(parent_name) if parent_name else self.model
                wrapper = LinearWithLoRA(module)
                setattr(parent, child, wrapper)
                self.lora_wrappers[name] = wrapper
        # "1": q/k/v fused for decode-shaped inputs (the reference's switch);
        # "all": for every input.  Gate/up: "1" or "all" fuses every input.
        fused_qkv = os.environ.get("MULTI_LORA_FUSED_QKV", "0")
        if fused_qkv in ("1", "all"):
            fuse_qkv_projections(self.lora_wrappers, all_shapes=fused_qkv == "all")
        if os.environ.get("MULTI_LORA_FUSED_GATE_UP", "0") in ("1", "all"):
            fuse_gate_up_projections(self.lora_wrappers)
        if os.environ.get("MULTI_LORA_FUSED_NORM", "1") == "1" and self.pool.device.type == "cuda":
            from .kernels.rmsnorm import fuse_rmsnorm

            fuse_rmsnorm(self.model)

    # -- per step --------------------------------------------------------------
    def prepare_lora_batch(self, lora_names: List[LoraName]) -> BatchLoRAInfo:
        if not validate_lora_batch(lora_names, max_loras_per_batch=self.max_loras_per_batch):
            raise ValueError(
                f"invalid lora batch: distinct={len(set(lora_names))} max={self.max_loras_per_batch}"
            )
        self.pool.prepare_lora_batch(dict.fromkeys(lora_names), weight_store=self._weight_store)
        return self.pool.build_batch_info(list(lora_names))

    @torch.inference_mode()
    def build_kernel_input_metadata(self, lora_names: List[LoraName], *, seq_lens: List[int]) -> KernelInputMetaData:
        names, lens = group_rows(lora_names, seq_lens)
        info = self.prepare_lora_batch(names)
        self._resident_meta = write_kernel_input_metadata(
            self._resident_meta, info, device=self.pool.device, dtype=self.pool.dtype, seq_lens=lens
        )
        return self._resident_meta

    def _setup_forward_batch(self, lora_names: List[LoraName], *, seq_lens: List[int]) -> None:
        meta = self.build_kernel_input_metadata(lora_names, seq_lens=seq_lens)
        self._lora_backend.set_kernel_input_metadata(meta)
        for key, wrapper in self.lora_wrappers.items():
            a, b = self.pool.get_module_buffers(key)
            wrapper.set_lora_info(self._lora_backend, a, b)

    @torch.inference_mode()
    def forward_with_lora(
        self,
        *,
        lora_names: List[LoraName],
        seq_lens: List[int],
        x: Optional[torch.Tensor] = None,
        input_ids: Optional[torch.Tensor] = None,
        attention_mask: Optional[torch.Tensor] = None,
        **kwargs,
    ):
        """Run the model with each row's adapter; ``seq_lens`` as in ``segment_lens``."""
        self._setup_forward_batch(lora_names, seq_lens=seq_lens)
        if x is not None:
            return self.model(x, **kwargs)
        if input_ids is None:
            raise ValueError("forward_with_lora requires input_ids or x")
        return self.model(input_ids=input_ids, attention_mask=attention_mask, **kwargs)

    def registered(self) -> Iterable[str]:
        return self._weight_store.keys()
