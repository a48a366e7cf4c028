"""Pool upload: one launch copies staged adapter banks into their slots.

``scatter_stage`` keeps the signature of the reference's
``scatter_stage(stage, slots, tables, total, h, rank, BLOCK=8192)``
(multi_lora/kernels/scatter_bank.py:68-93) and runs ``mlora_pool_scatter``:
for each staged row ``i < h`` and each module key, the bank's A block goes
into rows ``[0, rank)`` of ``A[key][slots[i]]`` and its B block into columns
``[0, rank)`` of ``B[key][slots[i]]``; nothing else in the pool changes.
``tables`` is what the pool's ``_RankPlan.build_tables`` returns for the
layout the banks were packed with.  There is no CPU path.
"""

from __future__ import annotations

import torch

from .. import _ffi
from .lora_ops import _int32, _require_gpu


def scatter_stage(stage: torch.Tensor, slots: torch.Tensor, tables: dict, total: int, h: int, rank: int,
                  BLOCK: int = 8192) -> None:  # noqa: N803 (the reference's keyword)
    """Scatter staged rows ``stage[:h]`` (each a packed bank of ``total``
    elements) into pool slots ``slots[:h]`` (int32 or int64, on the device).

    ``BLOCK`` is accepted for the reference's signature; the HIP kernel's
    block is fixed at 2048 elements, and any positive value gives the same
    result."""
    _require_gpu(stage, "stage")
    dev = stage.device
    if stage.dim() != 2 or stage.stride(1) != 1:
        raise ValueError("stage must be a 2-D [rows, total] tensor with contiguous rows")
    if not 0 <= h <= stage.shape[0]:
        raise ValueError(f"h={h} staged rows, but stage holds {stage.shape[0]}")
    if stage.shape[1] < total:
        raise ValueError(f"stage rows hold {stage.shape[1]} elements, fewer than the bank's {total}")
    if BLOCK <= 0:
        raise ValueError(f"BLOCK must be positive, got {BLOCK}")
    if slots.numel() < h:
        raise ValueError(f"{slots.numel()} slots for h={h} staged rows")
    if h == 0:
        return
    slots32 = _int32(slots.reshape(-1)[:h], dev)
    keys = tables["keys"]
    if keys.device != dev:
        raise ValueError(f"scatter tables are on {keys.device}, the stage on {dev}")
    rc = _ffi.lib().mlora_pool_scatter(
        stage.data_ptr(), stage.stride(0), int(h), slots32.data_ptr(), keys.data_ptr(), int(tables["n"]), int(rank),
        int(tables["num_slots"]), int(tables["max_numel"]), _ffi.dtype_code(stage.dtype), _ffi.stream_ptr(dev))
    _ffi.check(rc, "mlora_pool_scatter")
