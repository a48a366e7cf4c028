"""CPU restatement of the reference's LoRA shrink/expand (test infrastructure).

* ``TorchLoRABackend`` restates multi_lora/backend/torch_backend.py:17-90:
  a loop over segments; segment ``s`` covers rows ``[indptr[s], indptr[s+1])``
  (skipped if empty), uses slot ``weight_indices[s]`` and rank
  ``lora_ranks[slot]`` (skipped if 0); shrink computes
  ``y[rows, :r] = x[rows] @ A[slot, :r].T`` into a zero ``[S, r_max]``; expand
  adds ``(mid[rows, :r] @ B[slot, :, :r].T) * scalings[slot]`` into the output,
  all in ``x.dtype``.
* ``apply_f64`` is the brute-force closed form in float64 with no
  intermediate rounding: the ground truth for tolerance checks.
* ``apply_kernel_numerics`` restates the rounding sequence of the reference's
  GPU kernels (fp32 accumulate; ``mid`` rounded to the storage dtype,
  sgemm_lora_a.py:109; delta scaled in fp32 and rounded before the residual
  add, sgemm_lora_b.py:84-89), which the HIP kernels also follow.
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch

from multi_lora_amd.backend.base import LoRABackend
from multi_lora_amd.batch_info import KernelInputMetaData

Segment = Tuple[int, int, int, int, float]  # start, end, slot, rank, scaling


def segments(meta: KernelInputMetaData, rank_mult: int = 1, r_max: Optional[int] = None) -> List[Segment]:
    """Host view of the segment table: one tuple per non-empty, rank>0 segment."""
    bs = int(meta.bs)
    indptr = meta.seg_indptr.detach().cpu().tolist()
    widx = meta.weight_indices.detach().cpu().tolist()
    ranks = meta.lora_ranks.detach().cpu().tolist()
    scal = meta.scalings.detach().cpu().float().tolist()
    out: List[Segment] = []
    for s in range(bs):
        start, end = int(indptr[s]), int(indptr[s + 1])
        if start >= end:
            continue
        slot = int(widx[s])
        if slot < 0 or slot >= len(ranks):
            continue
        r = int(ranks[slot]) * rank_mult
        if r_max is not None:
            r = min(r, r_max)
        if r <= 0:
            continue
        out.append((start, end, slot, r, float(scal[slot])))
    return out


class TorchLoRABackend(LoRABackend):
    """Per-segment PyTorch path on host tensors (the reference's golden backend)."""

    name = "torch"

    def _meta(self) -> KernelInputMetaData:
        if self.kernel_input_metadata is None:
            raise RuntimeError("kernel_input_metadata not set; call set_kernel_input_metadata first")
        return self.kernel_input_metadata

    def run_lora_a_sgemm(self, x: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
        meta = self._meta()
        if x.dim() != 2:
            raise ValueError("TorchLoRABackend expects x [S, in]")
        y = torch.zeros(x.shape[0], weights.shape[1], device=x.device, dtype=x.dtype)
        for start, end, slot, r, _ in segments(meta):
            a = weights[slot, :r, :].to(dtype=x.dtype)
            y[start:end, :r] = x[start:end] @ a.T
        return y

    def run_lora_b_sgemm(
        self, x: torch.Tensor, weights: torch.Tensor, base_output: Optional[torch.Tensor] = None
    ) -> torch.Tensor:
        meta = self._meta()
        if x.dim() != 2:
            raise ValueError("TorchLoRABackend expects x [S, rank]")
        y = torch.zeros(x.shape[0], weights.shape[1], device=x.device, dtype=x.dtype) if base_output is None else base_output
        scal = meta.scalings
        for start, end, slot, r, _ in segments(meta):
            b = weights[slot, :, :r].to(dtype=x.dtype)
            scale = scal[slot].to(dtype=x.dtype)
            delta = (x[start:end, :r] @ b.T) * scale
            if base_output is None:
                y[start:end] = delta
            else:
                y[start:end] = y[start:end] + delta
        return y


def shrink_ref(x: torch.Tensor, a_stacks: Sequence[torch.Tensor], meta: KernelInputMetaData) -> torch.Tensor:
    """Multi-slice shrink in ``x.dtype``: slice ``s`` fills columns ``[s*r_max, s*r_max + r)``."""
    r_max = a_stacks[0].shape[1]
    y = torch.zeros(x.shape[0], len(a_stacks) * r_max, dtype=x.dtype)
    for start, end, slot, r, _ in segments(meta, r_max=r_max):
        for s, a in enumerate(a_stacks):
            y[start:end, s * r_max : s * r_max + r] = x[start:end] @ a[slot, :r].to(x.dtype).T
    return y


def lora_delta(x: torch.Tensor, lora_a: torch.Tensor, lora_b: torch.Tensor, scaling: float, *, rank: int) -> torch.Tensor:
    """``scaling * x @ A[:rank].T @ B[:, :rank].T`` (multi_lora/layers.py:23-39)."""
    flat = x.reshape(-1, x.shape[-1])
    d = (flat @ lora_a[:rank].T @ lora_b[:, :rank].T) * scaling
    return d.reshape(*x.shape[:-1], lora_b.shape[0])


def apply_f64(
    x: torch.Tensor,
    a_stacks: Sequence[torch.Tensor],
    b_stacks: Sequence[torch.Tensor],
    meta: KernelInputMetaData,
    base: torch.Tensor,
    col_offsets: Optional[Sequence[int]] = None,
) -> torch.Tensor:
    """Float64 ground truth: ``base + scaling * x A^T B^T`` per segment and slice, no rounding."""
    out = base.detach().cpu().double().clone()
    x64 = x.detach().cpu().double()
    if col_offsets is None:
        col_offsets = [0] * len(b_stacks) if len(b_stacks) == 1 else _consecutive(b_stacks)
    r_max = a_stacks[0].shape[1]
    for start, end, slot, r, sc in segments(meta, r_max=r_max):
        for a, b, c0 in zip(a_stacks, b_stacks, col_offsets):
            a64 = a[slot, :r].detach().cpu().double()
            b64 = b[slot, :, :r].detach().cpu().double()
            out[start:end, c0 : c0 + b.shape[1]] += sc * (x64[start:end] @ a64.T) @ b64.T
    return out


def _consecutive(b_stacks: Sequence[torch.Tensor]) -> List[int]:
    cols, c = [], 0
    for b in b_stacks:
        cols.append(c)
        c += b.shape[1]
    return cols


def _round(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return t.to(dtype).to(torch.float32)


def apply_kernel_numerics(
    x: torch.Tensor,
    a_stacks: Sequence[torch.Tensor],
    b_stacks: Sequence[torch.Tensor],
    meta: KernelInputMetaData,
    base: torch.Tensor,
    col_offsets: Optional[Sequence[int]] = None,
    shrink_input: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """The GPU kernels' rounding sequence on the CPU; returns ``(mid, out)`` in the storage dtype.

    fp32 accumulation in float64 here (the kernels' fp32 sums differ from it
    only in summation order), ``mid`` rounded to the storage dtype, delta
    scaled in fp32 and rounded, then added to the residual in fp32 and
    rounded again.  ``shrink_input``: float64 rows the shrink multiplies
    with A in place of x (the fused RMSNorm form's
    ``rmsnorm_ref.rmsnorm_shrink_input``); the storage dtype stays x's.
    """
    dt = x.dtype
    r_max = a_stacks[0].shape[1]
    if col_offsets is None:
        col_offsets = _consecutive(b_stacks)
    mid = torch.zeros(x.shape[0], len(a_stacks) * r_max, dtype=torch.float32)
    out = base.detach().cpu().float().clone()
    x64 = x.detach().cpu().double() if shrink_input is None else shrink_input.detach().cpu().double()
    for start, end, slot, r, sc in segments(meta, r_max=r_max):
        scale = float(torch.tensor(sc, dtype=torch.float32))
        for s, (a, b, c0) in enumerate(zip(a_stacks, b_stacks, col_offsets)):
            y = x64[start:end] @ a[slot, :r].detach().cpu().double().T
            y = _round(y.float(), dt)
            mid[start:end, s * r_max : s * r_max + r] = y
            d = (y.double() @ b[slot, :, :r].detach().cpu().double().T).float() * scale
            d = _round(d, dt)
            out[start:end, c0 : c0 + b.shape[1]] = _round(out[start:end, c0 : c0 + b.shape[1]] + d, dt)
    return mid.to(dt), out.to(dt)
