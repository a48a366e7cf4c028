"""LoRA compute backend interface (mirrors multi_lora/backend/base.py:13-89).

A backend holds the step's segment metadata and a reusable ``mid`` buffer
(stable address, sliced by rows) and computes ``A`` then ``B``:
``apply_lora(x, A_stack, B_stack, y)`` adds the LoRA delta of every segment
into ``y`` in place and returns it.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Optional

import torch

from ..batch_info import KernelInputMetaData


class LoRABackend(ABC):
    name: str = "abstract"

    def __init__(self) -> None:
        self.kernel_input_metadata: Optional[KernelInputMetaData] = None
        self._mid = torch.empty((0, 0))

    def mid_buffer(self, rows: int, max_rank: int, like: torch.Tensor) -> torch.Tensor:
        """A ``[rows, max_rank]`` scratch view, reused (same address) while it fits."""
        m = self._mid
        if m.shape[0] < rows or m.shape[1] != max_rank or m.device != like.device or m.dtype != like.dtype:
            self._mid = torch.empty((rows, max_rank), dtype=like.dtype, device=like.device)
        return self._mid[:rows]

    def set_kernel_input_metadata(self, metadata: KernelInputMetaData) -> None:
        self.kernel_input_metadata = metadata

    @abstractmethod
    def run_lora_a_sgemm(self, x: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
        """``x [S, in]`` with ``weights [K, r_max, in]`` -> ``mid [S, r_max]``."""

    @abstractmethod
    def run_lora_b_sgemm(
        self, x: torch.Tensor, weights: torch.Tensor, base_output: Optional[torch.Tensor] = None
    ) -> torch.Tensor:
        """``mid [S, r_max]`` with ``weights [K, out, r_max]``: scaled delta, added into ``base_output``."""

    def apply_lora(
        self, x: torch.Tensor, a_stack: torch.Tensor, b_stack: torch.Tensor, base_output: torch.Tensor
    ) -> torch.Tensor:
        """``base_output += scaling * (x @ A[slot,:r].T) @ B[slot,:,:r].T`` per segment."""
        mid = self.run_lora_a_sgemm(x, a_stack)
        return self.run_lora_b_sgemm(mid, b_stack, base_output=base_output)
