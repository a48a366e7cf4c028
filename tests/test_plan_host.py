"""The per-table plan on the host (CPU).

``batch_info.build_plan`` (vectorised numpy, the product's host builder) is
checked word for word against ``oracle.metadata_ref.plan_ref`` (plain
loops), and the oracle's row order against ``torch.argsort(stable=True)``
of the token slots, a library routine independent of both.  Tables cover
empty and ragged segments, slots outside the pool, rank-0 slots, segment
bounds past the call's rows, and plans too small for their table.
"""

import random

import numpy as np
import pytest
import torch

from multi_lora_amd.batch_info import (PLAN_ENTRY_WORDS, PLAN_HEADER_WORDS, PLAN_ROW_WORD, PLAN_ROWS, build_plan,
                                       plan_words)
from oracle.metadata_ref import plan_ref, slot_gather_order


def random_table(rng: random.Random):
    bs = rng.randint(0, 60)
    ns = rng.randint(1, 24)
    lens = [rng.choice([0, 1, 1, 1, 2, 3, 5, 16, 17, 40]) for _ in range(bs)]
    indptr = [0]
    for n in lens:
        indptr.append(indptr[-1] + n)
    slots = [rng.randint(-2, ns + 1) for _ in range(bs)]
    ranks = [rng.choice([0, 4, 8, 16]) for _ in range(ns)]
    scal = np.array([rng.uniform(0.1, 3.0) for _ in range(ns)], dtype=np.float32)
    rows = indptr[-1] if rng.random() < 0.7 else max(0, indptr[-1] - rng.randint(0, 10))
    return indptr, slots, ranks, scal, ns, rows


@pytest.mark.parametrize("seed", range(8))
def test_host_builder_matches_oracle(seed):
    rng = random.Random(seed)
    for _ in range(100):
        indptr, slots, ranks, scal, ns, rows = random_table(rng)
        cap = rng.randint(1, 64)
        out = np.zeros(plan_words(cap), np.int32)
        n = build_plan(indptr, slots, ranks, scal, ns, rows, out)
        ref = plan_ref(indptr, slots, ranks, scal.view(np.int32).tolist(), ns, rows, cap)
        assert n == ref[0]
        assert out.tolist() == ref


def test_gather_order_is_a_stable_sort_by_slot():
    """The plan's rows, entry by entry, are the live tokens stably sorted by slot."""
    rng = random.Random(99)
    for _ in range(200):
        indptr, slots, ranks, scal, ns, rows = random_table(rng)
        rows = indptr[-1]
        tok_slot = []
        for s in range(len(slots)):
            tok_slot.extend([slots[s]] * (indptr[s + 1] - indptr[s]))
        t = torch.tensor(tok_slot, dtype=torch.int64)
        live = torch.tensor([0 <= s < ns and ranks[s] > 0 for s in tok_slot], dtype=torch.bool)
        order = torch.argsort(t, stable=True)
        want = [int(i) for i in order if live[i]]
        cap = rows + 1
        words = plan_ref(indptr, slots, ranks, scal.view(np.int32).tolist(), ns, rows, cap)
        got = []
        for e in range(words[0]):
            base = PLAN_HEADER_WORDS + e * PLAN_ENTRY_WORDS
            got.extend(words[base + PLAN_ROW_WORD:base + PLAN_ROW_WORD + words[base + 3]])
        assert got == want
        assert words[1] == len(want)


def test_known_plan():
    """A table written out by hand: slots 2, 0, 2, 5 (rank 0), 0 with lengths 3, 1, 18, 2, 1."""
    indptr = [0, 3, 4, 22, 24, 25]
    slots = [2, 0, 2, 5, 0]
    ranks = [8, 8, 16, 0, 0, 0]
    scal = np.array([1.0, 1.0, 0.5, 1.0, 1.0, 2.0], np.float32)
    out = np.zeros(plan_words(8), np.int32)
    n = build_plan(indptr, slots, ranks, scal, 6, 25, out)
    assert n == 3  # slot 0: rows 3, 24; slot 2: rows 0-2 then 4-21 (21 rows -> 16 + 5)
    assert out[:3].tolist() == [3, 23, 8]
    e = out[PLAN_HEADER_WORDS:PLAN_HEADER_WORDS + 3 * PLAN_ENTRY_WORDS].reshape(3, PLAN_ENTRY_WORDS)
    assert e[:, :5].tolist() == [[0, 8, int(np.float32(1.0).view(np.int32)), 2, 0],
                                 [2, 16, int(np.float32(0.5).view(np.int32)), 16, 2],
                                 [2, 16, int(np.float32(0.5).view(np.int32)), 5, 18]]
    assert e[0, PLAN_ROW_WORD:PLAN_ROW_WORD + PLAN_ROWS].tolist() == [3, 24] + [3] * 14
    assert e[1, PLAN_ROW_WORD:PLAN_ROW_WORD + PLAN_ROWS].tolist() == [0, 1, 2] + list(range(4, 17))
    assert e[2, PLAN_ROW_WORD:PLAN_ROW_WORD + PLAN_ROWS].tolist() == list(range(17, 22)) + [17] * 11
    # slot_gather_order, the oracle's grouping underneath, agrees
    gslots, offs, toks = slot_gather_order(indptr, slots, ranks, len(slots))
    assert gslots == [0, 2] and offs == [0, 2, 23]


def test_planted_mistakes_fail_the_pins():
    """A plan that keeps rank-0 slots, splits at 15 rows or orders a slot's rows backwards differs."""
    indptr = [0, 3, 4, 22, 24, 25]
    slots = [2, 0, 2, 5, 0]
    ranks = [8, 8, 16, 0, 0, 0]
    bits = np.array([1.0] * 6, np.float32).view(np.int32).tolist()
    good = plan_ref(indptr, slots, ranks, bits, 6, 25, 8)
    assert plan_ref(indptr, slots, [8, 8, 16, 0, 0, 1], bits, 6, 25, 8) != good   # rank-0 slot 5 kept
    import oracle.metadata_ref as mr
    saved = mr.PLAN_ROWS
    try:
        mr.PLAN_ROWS = 15
        assert plan_ref(indptr, slots, ranks, bits, 6, 25, 8) != good
    finally:
        mr.PLAN_ROWS = saved
    # rows of a slot in descending order: the entry split then differs
    saved_order = mr.slot_gather_order
    try:
        def descending(*a, **k):
            gs, offs, toks = saved_order(*a, **k)
            return gs, offs, [t for g in range(len(gs)) for t in reversed(toks[offs[g]:offs[g + 1]])]
        mr.slot_gather_order = descending
        assert plan_ref(indptr, slots, ranks, bits, 6, 25, 8) != good
    finally:
        mr.slot_gather_order = saved_order
