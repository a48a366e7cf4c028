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
* ``build_plan``         the slot-grouped row lists of a table (no
                         counterpart in the reference; it lists, per
                         referenced slot, the rows that use it, in entries of
                         16), packed with the table so every call of a step
                         reuses it.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

# Segments of at most this many rows count as short (decode-like) in the
# table summary; the library's mixed-batch expand uses the same bound.
SHORT_SEG_ROWS = 16

# Plan layout (include/mlora_hip.h, MLORA_PLAN_*).
PLAN_HEADER_WORDS = 16
PLAN_ENTRY_WORDS = 32
PLAN_ROWS = 16
PLAN_ROW_WORD = 8


def plan_words(cap: int) -> int:
    """int32 words of a plan with room for ``cap`` entries."""
    return PLAN_HEADER_WORDS + cap * PLAN_ENTRY_WORDS


def build_plan(indptr, slots, ranks, scal_f32, num_slots: int, rows: int, out: np.ndarray) -> int:
    """Write the plan of a segment table into ``out`` (int32 words); returns its entry count.

    Entries take the slots in ascending order (slots outside
    ``[0, num_slots)`` and rank-0 slots excluded); each slot's rows, segment
    bounds clamped to ``[0, rows)``, in segment order, fill entries of 16:
    slot, rank, scaling (fp32 bits), row count, position of the first row
    among all planned rows, then the rows (unused words repeat the first).
    Entries past the room in ``out`` are left out; the header still counts
    them.  ``scal_f32``: each slot's scaling as the kernels read it (the
    pool dtype's value in fp32).
    """
    cap = (out.shape[0] - PLAN_HEADER_WORDS) // PLAN_ENTRY_WORDS
    ip = np.asarray(indptr, dtype=np.int64)
    w = np.asarray(slots, dtype=np.int64)
    rk = np.asarray(ranks, dtype=np.int64)[:num_slots]
    starts = np.clip(ip[:-1], 0, rows)
    ends = np.clip(ip[1:], 0, rows)
    inside = (w >= 0) & (w < num_slots)
    live = inside & (ends > starts)
    live[inside] &= rk[w[inside]] > 0
    lens = (ends - starts)[live]
    seg_slot = w[live]
    total = int(lens.sum())
    # Concatenated row ranges of the live segments, in segment order, then
    # stably grouped by slot.
    first = np.repeat(starts[live] - (np.cumsum(lens) - lens), lens)
    tok_rows = first + np.arange(total, dtype=np.int64)
    rows_sorted = tok_rows[np.argsort(np.repeat(seg_slot, lens), kind="stable")]
    slot_rows = np.bincount(seg_slot, weights=lens, minlength=num_slots).astype(np.int64)
    uniq = np.nonzero(slot_rows)[0]
    counts = slot_rows[uniq]
    n_ent = (counts + PLAN_ROWS - 1) // PLAN_ROWS
    n_entries = int(n_ent.sum())
    out[:PLAN_HEADER_WORDS] = 0
    out[0], out[1], out[2] = n_entries, total, cap
    e_take = min(n_entries, cap)
    if e_take:
        ent_slot = np.repeat(uniq, n_ent)[:e_take]
        k = (np.arange(n_entries) - np.repeat(np.cumsum(n_ent) - n_ent, n_ent))[:e_take]
        pos = np.repeat(np.cumsum(counts) - counts, n_ent)[:e_take] + PLAN_ROWS * k
        nr = np.minimum(PLAN_ROWS, np.repeat(counts, n_ent)[:e_take] - PLAN_ROWS * k)
        ent = out[PLAN_HEADER_WORDS:PLAN_HEADER_WORDS + e_take * PLAN_ENTRY_WORDS].reshape(e_take, PLAN_ENTRY_WORDS)
        ent[:] = 0
        ent[:, 0] = ent_slot
        ent[:, 1] = rk[ent_slot]
        ent[:, 2] = np.asarray(scal_f32, dtype=np.float32)[ent_slot].view(np.int32)
        ent[:, 3] = nr
        ent[:, 4] = pos
        i = np.arange(PLAN_ROWS)
        idx = pos[:, None] + np.where(i[None, :] < nr[:, None], i[None, :], 0)
        ent[:, PLAN_ROW_WORD:PLAN_ROW_WORD + PLAN_ROWS] = rows_sorted[idx]
    return n_entries


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
    # Set when the five columns are views of one device buffer with a pinned
    # host mirror (a GPU table made by write_kernel_input_metadata): a
    # rewrite is then one asynchronous copy instead of five.
    packed: Optional["PackedColumns"] = None
    # The table's plan (build_plan) when the table carries one: an int32
    # device tensor, its entry capacity and its entry count.  Packed tables
    # rebuild it on every rewrite; without one, the library builds it on the
    # device for each grouped call.
    plan: Optional[torch.Tensor] = None
    plan_cap: int = 0
    plan_entries: int = -1
    # Host copies of the segment lengths and slots (set by
    # write_kernel_input_metadata; None when unknown).  They give the
    # library a summary of the table (table_summary) with which a batch
    # mixing long and short segments gets one expand launch sized to it.
    host_lens: Optional[List[int]] = None
    host_slots: Optional[List[int]] = None
    _summaries: Dict[int, Tuple[int, int, int]] = field(default_factory=dict, repr=False, compare=False)

    def table_summary(self, num_slots: int) -> Tuple[int, int, int]:
        """(long_segs, long_rows, short_slots) for a pool of ``num_slots``
        slots, or (-1, -1, -1) without host copies: segments of more than 16
        rows and the rows they hold, and the distinct in-pool slots among the
        segments of 1 to 16 rows."""
        if self.host_lens is None or self.host_slots is None:
            return (-1, -1, -1)
        got = self._summaries.get(num_slots)
        if got is None:
            long_lens = [n for n in self.host_lens if n > SHORT_SEG_ROWS]
            short = {w for n, w in zip(self.host_lens, self.host_slots)
                     if 1 <= n <= SHORT_SEG_ROWS and 0 <= w < num_slots}
            got = self._summaries[num_slots] = (len(long_lens), sum(long_lens), len(short))
        return got

    def set_host_copies(self, lens: Sequence[int], slots: Sequence[int]) -> None:
        self.host_lens = list(lens)
        self.host_slots = list(slots)
        self._summaries.clear()


class PackedColumns:
    """One device buffer holding the five columns and the table's plan, and a pinned host mirror.

    Layout (each section 64-byte aligned): weight_indices[capacity],
    seg_lens[capacity], seg_indptr[capacity + 1] (int32), lora_ranks[num_slots]
    (int32), scalings[num_slots] (the pool dtype), then the plan (int32, room
    for capacity + min(capacity, num_slots) entries: every table of segments
    of at most 16 rows fits).  ``write`` fills the mirror, builds the plan in
    it, and copies everything up to the plan's last entry in one transfer on
    the current stream; before touching the mirror it waits for the previous
    transfer to have read it.
    """

    def __init__(self, capacity: int, num_slots: int, device: torch.device, dtype: torch.dtype) -> None:
        self.capacity, self.num_slots = capacity, num_slots
        self.plan_cap = max(1, capacity + min(capacity, num_slots))
        layout = [("weight_indices", capacity, torch.int32), ("seg_lens", capacity, torch.int32),
                  ("seg_indptr", capacity + 1, torch.int32), ("lora_ranks", num_slots, torch.int32),
                  ("scalings", num_slots, dtype), ("plan", plan_words(self.plan_cap), torch.int32)]
        offs, cur = [], 0
        for name, n, dt in layout:
            cur = (cur + 63) // 64 * 64
            offs.append((name, cur, n, dt))
            cur += n * torch.empty(0, dtype=dt).element_size()
        self.dev = torch.zeros(max(cur, 1), dtype=torch.uint8, device=device)
        self.host = torch.zeros(max(cur, 1), dtype=torch.uint8, pin_memory=True)
        self.dev_cols: Dict[str, torch.Tensor] = {}
        self.host_cols: Dict[str, torch.Tensor] = {}
        host_np = self.host.numpy()
        self.host_np = {}
        self.plan_off = offs[-1][1]
        self.plan_entries = 0
        for name, off, n, dt in offs:
            es = torch.empty(0, dtype=dt).element_size()
            self.dev_cols[name] = self.dev[off:off + n * es].view(dt)
            self.host_cols[name] = self.host[off:off + n * es].view(dt)
            if dt == torch.int32:
                self.host_np[name] = host_np[off:off + n * es].view(np.int32)
        self.event = torch.cuda.Event()
        self.pending = False

    def write(self, columns: Dict[str, Tuple[list, float]]) -> None:
        if self.pending:
            self.event.synchronize()
        rows = columns["seg_indptr"][0][-1] if columns["seg_indptr"][0] else 0
        for name, (values, pad) in columns.items():
            n = len(values)
            arr = self.host_np.get(name)
            if arr is not None:  # int32 columns: written through a numpy view of the pinned mirror
                arr[:n] = values
                arr[n:] = pad
                continue
            col = self.host_cols[name]
            if n:
                col[:n].copy_(torch.tensor(values, dtype=col.dtype))  # same conversion as fill_column
            col[n:].fill_(pad)
        np_cols = self.host_np
        nb = len(columns["weight_indices"][0])
        self.plan_entries = build_plan(
            np_cols["seg_indptr"][:nb + 1], np_cols["weight_indices"][:nb], np_cols["lora_ranks"],
            self.host_cols["scalings"].float().numpy(), self.num_slots, rows, np_cols["plan"])
        used = self.plan_off + 4 * plan_words(min(self.plan_entries, self.plan_cap))
        self.dev[:used].copy_(self.host[:used], non_blocking=True)
        self.event.record()
        self.pending = True


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
    A table allocated here on a GPU packs its columns into one buffer with a
    pinned host mirror, so each later rewrite is a single asynchronous copy
    (the reference issues one pageable copy per column, batch_info.py:153-157).
    """
    rows = len(pool_batch.weight_indices)
    lens, indptr = segment_lens(rows, seq_lens)
    max_len = max(lens) if lens else 0
    device = torch.device(device)
    slots = len(pool_batch.lora_ranks)
    columns = {
        "weight_indices": (list(pool_batch.weight_indices), 0),
        "seg_lens": (lens, 0),
        "seg_indptr": (indptr, indptr[-1]),
        "lora_ranks": (list(pool_batch.lora_ranks), 0),
        "scalings": (list(pool_batch.scalings), 0.0),
    }

    pk = meta.packed
    if pk is not None and rows <= pk.capacity and slots == pk.num_slots and meta.scalings.dtype == dtype:
        pk.write(columns)
        meta.bs = rows
        meta.max_len = max_len
        meta.plan_entries = pk.plan_entries
        meta.set_host_copies(lens, pool_batch.weight_indices)
        return meta

    if rows > meta.weight_indices.shape[0] or meta.packed is not None:
        if device.type == "cuda":
            pk = PackedColumns(rows, slots, device, dtype)
            pk.write(columns)
            c = pk.dev_cols
            fresh = KernelInputMetaData(bs=rows, seg_lens=c["seg_lens"], seg_indptr=c["seg_indptr"],
                                        weight_indices=c["weight_indices"], lora_ranks=c["lora_ranks"],
                                        scalings=c["scalings"], max_len=max_len, packed=pk, plan=c["plan"],
                                        plan_cap=pk.plan_cap, plan_entries=pk.plan_entries)
        else:
            fresh = KernelInputMetaData(
                bs=rows,
                seg_lens=torch.tensor(lens, dtype=torch.int32, device=device),
                seg_indptr=torch.tensor(indptr, dtype=torch.int32, device=device),
                weight_indices=torch.tensor(pool_batch.weight_indices, dtype=torch.int32, device=device),
                lora_ranks=torch.tensor(pool_batch.lora_ranks, dtype=torch.int32, device=device),
                scalings=torch.tensor(pool_batch.scalings, dtype=dtype, device=device),
                max_len=max_len,
            )
        fresh.set_host_copies(lens, pool_batch.weight_indices)
        return fresh

    fill_column(meta.weight_indices, pool_batch.weight_indices, 0)
    fill_column(meta.lora_ranks, pool_batch.lora_ranks, 0)
    fill_column(meta.seg_lens, lens, 0)
    fill_column(meta.seg_indptr, indptr, indptr[-1])
    fill_column(meta.scalings, pool_batch.scalings, 0.0)
    meta.bs = rows
    meta.max_len = max_len
    meta.set_host_copies(lens, pool_batch.weight_indices)
    return meta
