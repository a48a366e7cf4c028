"""Host-side adapter weights, the unit the slot pool uploads.

Same shape contract as the reference's ``AdapterWeights``
(multi_lora/weights.py:16-25): one rank and one scaling per adapter, and per
module key an ``A`` of shape ``[rank, in]`` and a ``B`` of shape ``[out, rank]``.
PEFT extraction (weights.py:36-68) is not part of this package; callers build
``AdapterWeights`` directly, with ``scaling = lora_alpha / rank`` as PEFT does.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Tuple

import torch

ModuleWeights = Dict[str, Tuple[torch.Tensor, torch.Tensor]]


@dataclass
class AdapterWeights:
    """All LoRA weights of one adapter (host tensors)."""

    rank: int
    scaling: float
    modules: ModuleWeights = field(default_factory=dict)
    # Set once the pool has packed the modules into its pinned upload bank and
    # released the per-module tensors.
    flattened: bool = False
    # Packed upload banks by (module layout, rank, dtype), filled by the pool.
    banks: Dict[tuple, torch.Tensor] = field(default_factory=dict, repr=False, compare=False)

    def validate(self) -> None:
        for key, (a, b) in self.modules.items():
            if a.dim() != 2 or b.dim() != 2:
                raise ValueError(f"{key}: A and B must be 2-D, got {tuple(a.shape)} and {tuple(b.shape)}")
            if a.shape[0] != self.rank or b.shape[1] != self.rank:
                raise ValueError(
                    f"{key}: A {tuple(a.shape)} / B {tuple(b.shape)} do not match rank {self.rank}"
                )
