"""Pins of the oracle's host logic against the reference's own known answers.

Each literal below is copied from the reference test or docstring cited next
to it; the oracle and the product restatement must both reproduce it.
"""

import pytest
import torch

from multi_lora_amd import batch_info as bi
from oracle.metadata_ref import group_rows_ref, resident_columns, segment_lens_ref, slot_gather_order, token_slots
from oracle.pool_ref import SlotPoolRef

GROUP_ROWS_CASES = [
    # multi_lora/tests/test_grouped_rows.py:32-37 (interleaved names do not merge)
    ((["a", "b", "a", "b"], []), (["a", "b", "a", "b"], [1, 1, 1, 1])),
    # test_grouped_rows.py:40-45 (adjacent names merge, None included)
    ((["a", "a", "b", "b", "b", None, None], []), (["a", "b", None], [2, 3, 2])),
    # test_grouped_rows.py:48-52 (prefill lengths add up)
    ((["a", "a", "b"], [5, 7, 3]), (["a", "b"], [12, 3])),
    # test_grouped_rows.py:137-156 (prefill rows [5,5,3,3] on a,a,b,b -> [10, 6])
    ((["a", "a", "b", "b"], [5, 5, 3, 3]), (["a", "b"], [10, 6])),
]


@pytest.mark.parametrize("args,expected", GROUP_ROWS_CASES)
@pytest.mark.parametrize("impl", [group_rows_ref, bi.group_rows], ids=["oracle", "product"])
def test_group_rows_known_answers(impl, args, expected):
    assert impl(*args) == expected


@pytest.mark.parametrize("impl", [group_rows_ref, bi.group_rows], ids=["oracle", "product"])
def test_group_rows_length_mismatch_raises(impl):
    # multi_lora/tests/test_grouped_rows.py:55-57
    with pytest.raises(ValueError):
        impl(["a", "b"], [1])


@pytest.mark.parametrize("impl", [segment_lens_ref, bi.segment_lens], ids=["oracle", "product"])
def test_segment_lens_known_answers(impl):
    # multi_lora/batch_info.py:48-49 docstring: decode and prefill examples
    assert impl(3, []) == ([1, 1, 1], [0, 1, 2, 3])
    assert impl(3, [13, 13, 22]) == ([13, 13, 22], [0, 13, 26, 48])
    assert impl(0, []) == ([], [0])


def test_group_rows_random_equivalence():
    g = torch.Generator().manual_seed(7)
    pool = ["a", "b", "c", None]
    for _ in range(200):
        n = int(torch.randint(0, 12, (1,), generator=g))
        names = [pool[int(i)] for i in torch.randint(0, 4, (n,), generator=g)]
        lens = [] if n % 2 else [int(v) for v in torch.randint(1, 9, (n,), generator=g)]
        assert bi.group_rows(names, lens) == group_rows_ref(names, lens)


def test_resident_metadata_rewrite_matches_oracle_padding():
    """In-place rewrite keeps addresses and pads each column as batch_info.py:169-178 does."""
    meta = bi.empty_kernel_input_metadata(device=torch.device("cpu"), dtype=torch.float32)
    info = bi.BatchLoRAInfo(weight_indices=[1, 0, 2, 1], lora_ranks=[4, 8, 0], scalings=[0.5, 2.0, 0.0])
    meta = bi.write_kernel_input_metadata(meta, info, device=torch.device("cpu"), dtype=torch.float32, seq_lens=[3, 1, 2, 5])
    ptrs = [meta.seg_indptr.data_ptr(), meta.weight_indices.data_ptr(), meta.lora_ranks.data_ptr()]
    small = bi.BatchLoRAInfo(weight_indices=[2, 0], lora_ranks=[4, 8, 1], scalings=[0.5, 2.0, 1.0])
    meta2 = bi.write_kernel_input_metadata(meta, small, device=torch.device("cpu"), dtype=torch.float32, seq_lens=[])
    assert meta2 is meta
    assert [meta.seg_indptr.data_ptr(), meta.weight_indices.data_ptr(), meta.lora_ranks.data_ptr()] == ptrs
    want = resident_columns([2, 0], [4, 8, 1], [0.5, 2.0, 1.0], [], capacity=4)
    assert meta.bs == 2 and meta.max_len == 1
    for col in ("weight_indices", "seg_lens", "seg_indptr", "lora_ranks", "scalings"):
        assert getattr(meta, col).tolist() == want[col], col
    # seg_indptr stays monotone through the padding
    ip = meta.seg_indptr.tolist()
    assert all(a <= b for a, b in zip(ip, ip[1:]))


# Literal columns after an in-place rewrite, worked out by hand from
# multi_lora/batch_info.py:169-176: every column keeps its length, unused
# segment slots get weight 0, length 0, indptr = the new total (so seg_indptr
# stays monotone), and lora_ranks / scalings (one per pool slot) are
# overwritten whole.
RESIDENT_PADDING_CASES = [
    # (first batch: weight_indices, seq_lens), (rewrite: weight_indices, ranks, scalings, seq_lens), expected
    (([1, 0, 2, 1], [3, 1, 2, 5]), ([2, 0], [4, 8, 1], [0.5, 2.0, 1.0], []),
     {"weight_indices": [2, 0, 0, 0], "seg_lens": [1, 1, 0, 0], "seg_indptr": [0, 1, 2, 2, 2],
      "lora_ranks": [4, 8, 1], "scalings": [0.5, 2.0, 1.0]}),
    (([0, 1, 2], []), ([1], [0, 16, 8], [0.0, 0.25, 4.0], [5]),
     {"weight_indices": [1, 0, 0], "seg_lens": [5, 0, 0], "seg_indptr": [0, 5, 5, 5],
      "lora_ranks": [0, 16, 8], "scalings": [0.0, 0.25, 4.0]}),
]


@pytest.mark.parametrize("first,rewrite,want", RESIDENT_PADDING_CASES)
def test_resident_padding_known_answer(first, rewrite, want):
    """The padding of an in-place rewrite, as literals: the oracle and the product both give them."""
    w0, lens0 = first
    w1, ranks, scal, lens1 = rewrite
    assert resident_columns(w1, ranks, scal, lens1, capacity=len(w0)) == want
    cpu = torch.device("cpu")
    meta = bi.empty_kernel_input_metadata(device=cpu, dtype=torch.float32)
    info0 = bi.BatchLoRAInfo(weight_indices=w0, lora_ranks=[8] * len(ranks), scalings=[1.0] * len(ranks))
    meta = bi.write_kernel_input_metadata(meta, info0, device=cpu, dtype=torch.float32, seq_lens=lens0)
    info1 = bi.BatchLoRAInfo(weight_indices=w1, lora_ranks=ranks, scalings=scal)
    assert bi.write_kernel_input_metadata(meta, info1, device=cpu, dtype=torch.float32, seq_lens=lens1) is meta
    for col, v in want.items():
        assert getattr(meta, col).tolist() == v, col
    assert meta.bs == len(w1) and meta.max_len == max(lens1 or [1])


def test_metadata_shapes_known_answer():
    # multi_lora/tests/test_phase4_backend.py:85-95: two decode rows [a, None]
    # in a 3-slot pool -> bs 2, seg_indptr[:3] == [0, 1, 2], one rank per slot.
    info = bi.BatchLoRAInfo(weight_indices=[0, 1], lora_ranks=[4, 0, 0], scalings=[2.0, 0.0, 0.0])
    meta = bi.write_kernel_input_metadata(
        bi.empty_kernel_input_metadata(device=torch.device("cpu"), dtype=torch.float32),
        info, device=torch.device("cpu"), dtype=torch.float32, seq_lens=[1, 1])
    assert meta.bs == 2
    assert meta.weight_indices.shape[0] >= meta.bs
    assert meta.lora_ranks.shape[0] == 3
    assert meta.seg_indptr[:3].tolist() == [0, 1, 2]


def test_lru_known_answer_oracle():
    # multi_lora/tests/test_pool.py:16-52: 2 slots, {a, b} then {c, None}
    # evicts both a and b.
    ref = SlotPoolRef(2, "lru")
    ref.prepare(["a", "b"])
    assert set(ref.slot_of) == {"a", "b"}
    ref.prepare(["c", None])
    assert set(ref.slot_of) == {"c", None}
    assert ref.evictions >= 1


def test_lru_versus_fifo_order_oracle():
    # Closed-form consequence of the two policies (multi_lora/eviction.py:26-35):
    # after a,b,c fill 3 slots and a is used again, LRU evicts b but FIFO evicts a.
    for kind, victim in (("lru", "b"), ("fifo", "a")):
        ref = SlotPoolRef(3, kind)
        for n in ("a", "b", "c"):
            ref.prepare([n])
        ref.prepare(["a"])
        ref.prepare(["d"])
        assert victim not in ref.slot_of, kind
        assert "d" in ref.slot_of


def test_base_evicted_last_oracle():
    ref = SlotPoolRef(2, "lru")
    ref.prepare([None])
    ref.prepare(["a"])
    ref.prepare(["b"])  # a is the only queued adapter not in the batch
    assert set(ref.slot_of) == {None, "b"}
    ref.prepare(["c", "b"])  # nothing queued is free: the base slot goes
    assert set(ref.slot_of) == {"b", "c"}
    with pytest.raises(ValueError):
        ref.prepare(["x", "y", "z"])


def test_token_slots_and_gather_order_brute_force():
    g = torch.Generator().manual_seed(3)
    for _ in range(50):
        bs = int(torch.randint(1, 20, (1,), generator=g))
        lens = torch.randint(0, 5, (bs,), generator=g).tolist()
        slots = torch.randint(-1, 6, (bs,), generator=g).tolist()
        ranks = torch.randint(0, 3, (6,), generator=g).tolist()
        indptr = [0]
        for n in lens:
            indptr.append(indptr[-1] + n)
        ts = token_slots(indptr, slots, bs)
        assert ts == torch.repeat_interleave(torch.tensor(slots, dtype=torch.long), torch.tensor(lens)).tolist()
        gslots, offs, toks = slot_gather_order(indptr, slots, ranks, bs)
        # brute force: stable sort of live tokens by slot
        live = [t for t in range(len(ts)) if 0 <= ts[t] < 6 and ranks[ts[t]] > 0]
        order = sorted(live, key=lambda t: (ts[t], t))
        assert toks == order
        assert gslots == sorted({ts[t] for t in live})
        for gi, s in enumerate(gslots):
            assert all(ts[t] == s for t in toks[offs[gi]:offs[gi + 1]])
