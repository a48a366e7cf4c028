"""Per-step segment metadata: host list form and resident device form.

Mirrors multi_lora/batch_info.py:16-179 (same names, fields and padding
rules) so callers of the reference can switch without edits:

* ``BatchLoRAInfo``      host lists from the pool: slot per row, rank and
                         scaling per slot (batch_info.py:16-22).
* ``KernelInputMetaData`` device tensors the kernels read (batch_info.py:25-42).
* ``segment_lens``       lengths + exclusive prefix sum (batch_info.py:45-67).
* ``group_rows``         run-length merge of adjacent equal names (:70-97).
* ``write_kernel_input_metadata`` rewrites resident tensors in place when
  they are large enough, so addresses stay fixed across steps (:128-179).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Sequence, Tuple

import torch


@dataclass
class BatchLoRAInfo:
    """Slot assignment of one batch (host lists)."""

    weight_indices: List[int]  # one per segment: its pool slot
    lora_ranks: List[int]  # one per slot: its rank (0 = base / empty)
    scalings: List[float]  # one per slot: its scaling


@dataclass
class KernelInputMetaData:
    """Device-side segment table read by the shrink/expand kernels.

    Segment ``s`` owns flattened rows ``[seg_indptr[s], seg_indptr[s+1])`` and
    uses slot ``weight_indices[s]``; ``lora_ranks`` / ``scalings`` are indexed
    by slot.  ``bs`` and ``max_len`` are host ints that size the launch grid.
    """

    bs: int
    seg_lens: torch.Tensor
    seg_indptr: torch.Tensor
    weight_indices: torch.Tensor
    lora_ranks: torch.Tensor
    scalings: torch.Tensor
    max_len: int


def segment_lens(bs: int, seq_lens: Sequence[int]) -> Tuple[List[int], List[int]]:
    """Per-segment token counts and their exclusive prefix sum.

    ``seq_lens == []`` means decode: every one of the ``bs`` segments has one
    token.  Otherwise ``seq_lens`` gives each segment's length and must have
    ``bs`` entries.  ``indptr`` has ``bs + 1`` entries, starting at 0.
    """
    if len(seq_lens) == 0:
        lens = [1 for _ in range(bs)]
    else:
        assert len(seq_lens) == bs, f"seq_lens has {len(seq_lens)} entries for {bs} segments"
        lens = [int(n) for n in seq_lens]
    indptr = [0] * (len(lens) + 1)
    for i, n in enumerate(lens):
        indptr[i + 1] = indptr[i] + n
    return lens, indptr


def group_rows(names: list, seq_lens: Sequence[int]) -> Tuple[list, List[int]]:
    """Merge runs of adjacent rows that use the same adapter into one segment.

    Only neighbours are merged and row order is kept, so KV-cache row
    alignment is untouched.  Decode (``seq_lens == []``) counts one token per
    row; prefill sums the rows' token counts.  Raises ``ValueError`` if
    ``seq_lens`` is given with a different length than ``names``.
    """
    counts = [1] * len(names) if len(seq_lens) == 0 else [int(n) for n in seq_lens]
    if len(counts) != len(names):
        raise ValueError(f"seq_lens ({len(counts)}) must have the same length as names ({len(names)})")
    out_names: list = []
    out_lens: List[int] = []
    prev = object()  # sentinel that equals no name, including None
    for name, n in zip(names, counts):
        if out_names and name == prev:
            out_lens[-1] += n
        else:
            out_names.append(name)
            out_lens.append(n)
        prev = name
    return out_names, out_lens


def fill_column(column: torch.Tensor, values: list, pad: float) -> None:
    """Overwrite a resident column in place: ``values`` then ``pad`` to the end.

    The tensor object, its length and its device address are unchanged.
    """
    size = column.shape[0]
    assert len(values) <= size, f"{len(values)} values do not fit in {size} entries"
    full = list(values)
    full.extend([pad] * (size - len(values)))
    column.copy_(torch.tensor(full, dtype=column.dtype))


def empty_kernel_input_metadata(*, device: torch.device, dtype: torch.dtype) -> KernelInputMetaData:
    """Zero-capacity metadata; the first write allocates real tensors."""

    def i32() -> torch.Tensor:
        return torch.empty(0, dtype=torch.int32, device=device)

    return KernelInputMetaData(
        bs=0,
        seg_lens=i32(),
        seg_indptr=i32(),
        weight_indices=i32(),
        lora_ranks=i32(),
        scalings=torch.empty(0, dtype=dtype, device=device),
        max_len=0,
    )


def write_kernel_input_metadata(
    meta: KernelInputMetaData,
    pool_batch: BatchLoRAInfo,
    *,
    device: torch.device,
    dtype: torch.dtype,
    seq_lens: Sequence[int],
) -> KernelInputMetaData:
    """Write this batch's segment table; in place when capacity allows.

    Returns ``meta`` itself (same tensors, same addresses) when its capacity
    holds the batch, which keeps graph-captured launches valid; otherwise a
    newly allocated table sized for this batch.  Unused tail entries are
    padded so every column is self-consistent: slot 0, rank 0, length 0,
    ``seg_indptr`` = total rows (monotone), scaling 0.
    ``lora_ranks`` / ``scalings`` always have one entry per pool slot.
    """
    rows = len(pool_batch.weight_indices)
    lens, indptr = segment_lens(rows, seq_lens)
    max_len = max(lens) if lens else 0

    if rows > meta.weight_indices.shape[0]:
        return KernelInputMetaData(
            bs=rows,
            seg_lens=torch.tensor(lens, dtype=torch.int32, device=device),
            seg_indptr=torch.tensor(indptr, dtype=torch.int32, device=device),
            weight_indices=torch.tensor(pool_batch.weight_indices, dtype=torch.int32, device=device),
            lora_ranks=torch.tensor(pool_batch.lora_ranks, dtype=torch.int32, device=device),
            scalings=torch.tensor(pool_batch.scalings, dtype=dtype, device=device),
            max_len=max_len,
        )

    fill_column(meta.weight_indices, pool_batch.weight_indices, 0)
    fill_column(meta.lora_ranks, pool_batch.lora_ranks, 0)
    fill_column(meta.seg_lens, lens, 0)
    fill_column(meta.seg_indptr, indptr, indptr[-1])
    fill_column(meta.scalings, pool_batch.scalings, 0.0)
    meta.bs = rows
    meta.max_len = max_len
    return meta
