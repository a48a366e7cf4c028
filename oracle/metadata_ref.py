"""CPU restatement of the segment-table logic (test infrastructure).

Follows multi_lora/batch_info.py:45-179 in behaviour, written independently:

* ``segment_lens_ref``   — lengths and exclusive prefix sum (batch_info.py:45-67);
* ``group_rows_ref``     — run-length merge of adjacent equal names (batch_info.py:70-97);
* ``resident_columns``   — what each resident column holds after an in-place
                           rewrite, padding included (batch_info.py:169-178);
* ``token_slots``        — slot of every token: ``repeat_interleave(weight_indices, seg_lens)``;
* ``slot_gather_order``  — tokens grouped by slot, stable within a slot;
* ``plan_ref``           — the per-table plan the decode kernels follow
                           (include/mlora_hip.h, MLORA_PLAN_*): the gather
                           order cut into entries of 16 rows.  It has no
                           counterpart in the reference; it regroups
                           ``slot_gather_order``, which the reference's
                           batch metadata implies (batch_info.py:128-179).
"""

from __future__ import annotations

import itertools
from typing import Dict, List, Sequence, Tuple


def segment_lens_ref(bs: int, seq_lens: Sequence[int]) -> Tuple[List[int], List[int]]:
    lens = [1] * bs if not seq_lens else [int(v) for v in seq_lens]
    if seq_lens:
        assert len(lens) == bs
    return lens, [0] + list(itertools.accumulate(lens))


def group_rows_ref(names: list, seq_lens: Sequence[int]) -> Tuple[list, List[int]]:
    counts = [1] * len(names) if not seq_lens else [int(v) for v in seq_lens]
    if len(counts) != len(names):
        raise ValueError("seq_lens and names differ in length")
    out_names, out_lens = [], []
    # groupby over indices keyed by name merges exactly the adjacent runs.
    for name, run in itertools.groupby(range(len(names)), key=lambda i: names[i]):
        out_names.append(name)
        out_lens.append(sum(counts[i] for i in run))
    return out_names, out_lens


def resident_columns(
    weight_indices: List[int], lora_ranks: List[int], scalings: List[float], seq_lens: Sequence[int], capacity: int
) -> Dict[str, list]:
    """Column contents after an in-place metadata rewrite of a table with ``capacity`` segments."""
    lens, indptr = segment_lens_ref(len(weight_indices), seq_lens)
    pad = capacity - len(weight_indices)
    return {
        "weight_indices": list(weight_indices) + [0] * pad,
        "seg_lens": lens + [0] * pad,
        "seg_indptr": indptr + [indptr[-1]] * pad,
        "lora_ranks": list(lora_ranks),
        "scalings": list(scalings),
    }


def token_slots(indptr: Sequence[int], weight_indices: Sequence[int], bs: int) -> List[int]:
    out: List[int] = []
    for s in range(bs):
        out.extend([int(weight_indices[s])] * (int(indptr[s + 1]) - int(indptr[s])))
    return out


def slot_gather_order(
    indptr: Sequence[int], weight_indices: Sequence[int], lora_ranks: Sequence[int], bs: int
) -> Tuple[List[int], List[int], List[int]]:
    """Tokens of rank>0 slots grouped by slot (ascending slot, ascending token).

    Returns ``(group_slots, group_offsets, tokens)``: group ``g`` is slot
    ``group_slots[g]`` and owns ``tokens[group_offsets[g]:group_offsets[g+1]]``.
    """
    per_slot: Dict[int, List[int]] = {}
    for s in range(bs):
        slot = int(weight_indices[s])
        if slot < 0 or slot >= len(lora_ranks) or int(lora_ranks[slot]) <= 0:
            continue
        per_slot.setdefault(slot, []).extend(range(int(indptr[s]), int(indptr[s + 1])))
    slots = sorted(k for k, v in per_slot.items() if v)
    offsets, tokens = [0], []
    for slot in slots:
        tokens.extend(per_slot[slot])
        offsets.append(len(tokens))
    return slots, offsets, tokens


PLAN_HEADER_WORDS, PLAN_ENTRY_WORDS, PLAN_ROWS, PLAN_ROW_WORD = 16, 32, 16, 8


def plan_ref(indptr: Sequence[int], weight_indices: Sequence[int], lora_ranks: Sequence[int],
             scal_bits: Sequence[int], num_slots: int, rows: int, cap: int) -> List[int]:
    """The plan's int32 words for a table, by plain loops.

    Segment bounds are clamped to ``[0, rows)``; slots outside
    ``[0, num_slots)`` and rank-0 slots get no entry.  ``scal_bits``: each
    slot's scaling as fp32 bit patterns (int).  Entries past ``cap`` are not
    written, but the header counts them.
    """
    bs = len(weight_indices)
    cl = [min(max(int(v), 0), rows) for v in indptr]
    ranks = [int(r) for r in lora_ranks[:num_slots]]
    slots, offsets, tokens = slot_gather_order(cl, weight_indices, ranks, bs)
    words = [0] * (PLAN_HEADER_WORDS + cap * PLAN_ENTRY_WORDS)
    e = 0
    for g, slot in enumerate(slots):
        mine = tokens[offsets[g]:offsets[g + 1]]
        for k in range(0, len(mine), PLAN_ROWS):
            part = mine[k:k + PLAN_ROWS]
            if e < cap:
                base = PLAN_HEADER_WORDS + e * PLAN_ENTRY_WORDS
                words[base + 0] = slot
                words[base + 1] = ranks[slot]
                words[base + 2] = int(scal_bits[slot])
                words[base + 3] = len(part)
                words[base + 4] = offsets[g] + k
                for i in range(PLAN_ROWS):
                    words[base + PLAN_ROW_WORD + i] = part[i] if i < len(part) else part[0]
            e += 1
    words[0], words[1], words[2] = e, len(tokens), cap
    return words
