"""The MI355X backend: every LoRA computation runs in libmlora_hip.

Drop-in for the reference's GPU backend (multi_lora/backend/triton_backend.py:19-78)
with the same methods and the same int32 coercion of the segment table, but
with no fallback: a CPU tensor or a missing library raises.  Besides the
reference's ``run_lora_a_sgemm`` / ``run_lora_b_sgemm`` / ``apply_lora`` it
offers ``apply_lora_multi`` for fused projections (q|k|v, gate|up): one
shrink that reads x once and one expand over all slices, and
``rmsnorm_apply_lora_multi``, which folds the RMSNorm in front of such a
projection into the LoRA shrink's launch.
"""

from __future__ import annotations

from typing import Callable, List, Optional, Sequence

import torch

from ..kernels.lora_ops import (GROUPED_MAX_LEN, LinkedWorkspace, Workspace, apply_grouped, apply_segments, expand,
                                 rmsnorm_apply_grouped, shrink)
from ..kernels.rmsnorm import rmsnorm_fwd
from .base import LoRABackend


class HipLoRABackend(LoRABackend):
    name = "hip"

    def __init__(self) -> None:
        super().__init__()
        self.workspace = Workspace()
        self.linked_workspace = LinkedWorkspace()

    def _meta(self):
        if self.kernel_input_metadata is None:
            raise RuntimeError("kernel_input_metadata not set; call set_kernel_input_metadata first")
        return self.kernel_input_metadata

    def run_lora_a_sgemm(self, x: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
        meta = self._meta()
        if x.dim() != 2:
            raise ValueError("HipLoRABackend expects x [S, in]")
        out = self.mid_buffer(x.shape[0], weights.shape[-2], x)
        return shrink(x.contiguous(), [weights.contiguous()], meta, out, workspace=self.workspace)

    def run_lora_b_sgemm(
        self, x: torch.Tensor, weights: torch.Tensor, base_output: Optional[torch.Tensor] = None
    ) -> torch.Tensor:
        meta = self._meta()
        if x.dim() != 2:
            raise ValueError("HipLoRABackend expects x [S, rank]")
        if base_output is None:
            base_output = torch.zeros((x.shape[0], weights.shape[-2]), device=x.device, dtype=x.dtype)
        return expand(x.contiguous(), [weights.contiguous()], meta, base_output, [0])

    def apply_lora(
        self, x: torch.Tensor, a_stack: torch.Tensor, b_stack: torch.Tensor, base_output: torch.Tensor
    ) -> torch.Tensor:
        """Add each segment's LoRA delta into ``base_output`` (in place) and return it.

        Decode-shaped batches (every segment at most 16 rows) take the
        slot-grouped path, which reads each referenced adapter once per call;
        other batches run the segment shrink and expand in one library call.
        """
        return self.apply_lora_multi(x, [a_stack], [b_stack], base_output, [0])

    def apply_lora_multi(
        self,
        x: torch.Tensor,
        a_stacks: Sequence[torch.Tensor],
        b_stacks: Sequence[torch.Tensor],
        base_output: torch.Tensor,
        col_offsets: Optional[List[int]] = None,
    ) -> torch.Tensor:
        """Add every slice's delta into its column range of ``base_output``.

        Slice ``s`` uses ``a_stacks[s]`` / ``b_stacks[s]`` and writes columns
        ``[col_offsets[s], col_offsets[s] + out_s)`` (default: consecutive).
        Equal to ``apply_lora`` per slice on the column views, element for element.
        """
        meta = self._meta()
        if x.dim() != 2:
            raise ValueError("HipLoRABackend expects x [S, in]")
        if col_offsets is None:
            col_offsets, c = [], 0
            for b in b_stacks:
                col_offsets.append(c)
                c += b.shape[1]
        x = x.contiguous()
        a_stacks = [a.contiguous() for a in a_stacks]
        b_stacks = [b.contiguous() for b in b_stacks]
        if meta.max_len <= GROUPED_MAX_LEN and apply_grouped(
            x, a_stacks, b_stacks, meta, base_output, col_offsets, workspace=self.linked_workspace,
        ):
            return base_output
        return apply_segments(x, a_stacks, b_stacks, meta, base_output, col_offsets, workspace=self.workspace)

    def rmsnorm_apply_lora_multi(
        self,
        x: torch.Tensor,
        weight: torch.Tensor,
        eps: float,
        a_stacks: Sequence[torch.Tensor],
        b_stacks: Sequence[torch.Tensor],
        base_output: torch.Tensor,
        col_offsets: Optional[List[int]] = None,
        base_fn: Optional[Callable[[torch.Tensor, torch.Tensor], None]] = None,
    ) -> torch.Tensor:
        """``y = RMSNorm(x)``, then ``base_fn(y, base_output)`` if given (the
        base projection writing ``base_output``), then every slice's LoRA
        delta of ``y`` added into ``base_output``; returns ``y``.

        Decode-shaped batches run the RMSNorm inside the LoRA shrink's launch
        (``mlora_rmsnorm_apply_grouped``: x read once, no RMSNorm launch of
        its own, y the same bits as ``rmsnorm_fwd``); the delta then differs
        from LoRA on y only in the rounding of the shrink's inputs.  Other
        batches run ``rmsnorm_fwd`` and ``apply_lora_multi``.
        """
        meta = self._meta()
        if x.dim() != 2:
            raise ValueError("HipLoRABackend expects x [S, in]")
        if col_offsets is None:
            col_offsets, c = [], 0
            for b in b_stacks:
                col_offsets.append(c)
                c += b.shape[1]
        x = x.contiguous()
        a_stacks = [a.contiguous() for a in a_stacks]
        b_stacks = [b.contiguous() for b in b_stacks]
        y = torch.empty_like(x)
        args = (x, weight, eps, y, a_stacks, b_stacks, meta, base_output, col_offsets, self.linked_workspace)
        if meta.max_len <= GROUPED_MAX_LEN and rmsnorm_apply_grouped(*args, phases=1):
            if base_fn is not None:
                base_fn(y, base_output)
            rmsnorm_apply_grouped(*args, phases=2)
            return y
        y = rmsnorm_fwd(x, weight, eps)
        if base_fn is not None:
            base_fn(y, base_output)
        self.apply_lora_multi(y, a_stacks, b_stacks, base_output, col_offsets)
        return y
