"""The product slot pool's host logic on CPU tensors, against the oracle.

Slot choice and eviction follow multi_lora/pool.py:382-473 and
multi_lora/eviction.py:12-50 (oracle: ``oracle/pool_ref.py``, itself pinned
by the reference's known answers in test_oracle_known_answers.py); slot
contents follow multi_lora/pool.py:234-244: only the first ``rank`` rows of
A and columns of B are written, the rest of the slot is zero.
"""

import random

import pytest
import torch

from multi_lora_amd import AdapterWeights, LoRAMemoryPool
from oracle.pool_ref import SlotPoolRef

DIMS = {"q_proj": (24, 40), "v_proj": (24, 16)}  # key -> (in, out)


def adapter(seed: int, rank: int, keys=("q_proj", "v_proj")) -> AdapterWeights:
    g = torch.Generator().manual_seed(seed)
    mods = {}
    for k in keys:
        i, o = DIMS[k]
        mods[k] = (torch.randn(rank, i, generator=g), torch.randn(o, rank, generator=g))
    return AdapterWeights(rank=rank, scaling=2.0 / rank, modules=mods)


def store(n: int):
    return {f"a{i}": adapter(i, [2, 4, 8][i % 3]) for i in range(n)}


@pytest.mark.parametrize("policy", ["lru", "fifo"])
def test_slot_assignment_matches_oracle_random_batches(policy):
    rng = random.Random(5)
    names = [f"a{i}" for i in range(12)] + [None]
    st = store(12)
    k = 5
    pool = LoRAMemoryPool(k, 8, torch.device("cpu"), torch.float32, eviction_policy=policy)
    ref = SlotPoolRef(k, policy)
    for _ in range(60):
        batch = [rng.choice(names) for _ in range(rng.randint(1, k))]
        batch = list(dict.fromkeys(batch))
        pool.prepare_lora_batch(batch, weight_store=st)
        ref.prepare(batch)
        assert {n: pool.get_slot_id(n) for n in batch} == {n: ref.slot_of[n] for n in batch}
        assert dict(pool.name_to_slot) == dict(ref.slot_of)


def test_slot_contents_are_rank_prefixes_and_zero_elsewhere():
    st = store(4)
    pool = LoRAMemoryPool(4, 8, torch.device("cpu"), torch.float32)
    pool.prepare_lora_batch(["a0", "a1", None, "a2"], weight_store=st)
    info = pool.build_batch_info(["a2", "a0", None, "a1"])
    for key, (i, o) in DIMS.items():
        a_stack, b_stack = pool.get_module_buffers(key)
        assert tuple(a_stack.shape) == (4, 8, i) and tuple(b_stack.shape) == (4, o, 8)
        for name in ("a0", "a1", "a2"):
            s = pool.get_slot_id(name)
            w = st[name]
            a, b = w.modules[key] if not w.flattened else (None, None)
            r = w.rank
            if a is not None:
                assert torch.equal(a_stack[s, :r], a) and torch.equal(b_stack[s, :, :r], b)
            assert not a_stack[s, r:].any() and not b_stack[s, :, r:].any()
        base = pool.get_slot_id(None)
        assert not a_stack[base].any() and not b_stack[base].any()
    assert info.weight_indices == [pool.get_slot_id(n) for n in ["a2", "a0", None, "a1"]]
    for name in ("a0", "a1", "a2"):
        s = pool.get_slot_id(name)
        assert info.lora_ranks[s] == st[name].rank
        assert info.scalings[s] == pytest.approx(st[name].scaling)
    assert info.lora_ranks[pool.get_slot_id(None)] == 0 and info.scalings[pool.get_slot_id(None)] == 0.0


def test_reused_slot_rewrites_the_rank_prefix_only():
    """A rank-2 adapter taking the slot of a rank-8 one overwrites rows [:2]
    of A and columns [:2] of B; the rows past its rank keep the old adapter's
    values, as the reference's slot write does (multi_lora/pool.py:234-244).
    Kernels never read past the rank (GPU tests with stale tails)."""
    st = {"big": adapter(1, 8), "small": adapter(2, 2), "x": adapter(3, 4)}
    pool = LoRAMemoryPool(2, 8, torch.device("cpu"), torch.float32)
    pool.prepare_lora_batch(["big", "x"], weight_store=st)
    slot = pool.get_slot_id("big")
    a_stack, b_stack = pool.get_module_buffers("q_proj")
    old_a, old_b = a_stack[slot].clone(), b_stack[slot].clone()
    pool.prepare_lora_batch(["x", "small"], weight_store=st)
    assert pool.get_slot_id("small") == slot
    a_new, b_new = adapter(2, 2).modules["q_proj"]
    assert torch.equal(a_stack[slot, :2], a_new) and torch.equal(b_stack[slot, :, :2], b_new)
    assert torch.equal(a_stack[slot, 2:], old_a[2:]) and torch.equal(b_stack[slot, :, 2:], old_b[:, 2:])
    assert pool.build_batch_info(["small"]).lora_ranks[slot] == 2


def test_missing_module_key_zeroes_the_slot_for_that_module():
    """An adapter without a v_proj delta contributes nothing to v_proj."""
    st = {"full": adapter(1, 4), "qonly": adapter(2, 4, keys=("q_proj",))}
    pool = LoRAMemoryPool(1, 8, torch.device("cpu"), torch.float32)
    pool.prepare_lora_batch(["full"], weight_store=st)
    pool.prepare_lora_batch(["qonly"], weight_store=st)
    a_stack, b_stack = pool.get_module_buffers("v_proj")
    assert not a_stack[0].any() and not b_stack[0].any()


def test_batch_larger_than_pool_raises():
    st = store(3)
    pool = LoRAMemoryPool(2, 8, torch.device("cpu"), torch.float32)
    with pytest.raises(ValueError):
        pool.prepare_lora_batch(["a0", "a1", "a2"], weight_store=st)


def test_rank_above_pool_max_raises():
    st = {"wide": adapter(1, 8)}
    pool = LoRAMemoryPool(2, 4, torch.device("cpu"), torch.float32)
    with pytest.raises(ValueError):
        pool.prepare_lora_batch(["wide"], weight_store=st)


def test_bank_is_packed_once_and_kept_on_the_adapter():
    """Packing follows the layout (every A block, then every B block); a
    reload reuses the adapter's bank, and a second pool with the same module
    layout reuses it too."""
    st = {"a": adapter(1, 4), "b": adapter(2, 4), "c": adapter(3, 4)}
    a_mods = {k: (a.clone(), b.clone()) for k, (a, b) in st["a"].modules.items()}
    pool = LoRAMemoryPool(2, 8, torch.device("cpu"), torch.float32)
    pool.prepare_lora_batch(["a"], weight_store=st)
    (bank,) = st["a"].banks.values()
    plan = pool.buffers.layout(4)
    want = torch.cat([a_mods[k][0].reshape(-1) for k in plan.keys] + [a_mods[k][1].reshape(-1) for k in plan.keys])
    assert torch.equal(bank, want)
    assert st["a"].flattened and not st["a"].modules
    pool.prepare_lora_batch(["b", "c"], weight_store=st)   # evicts "a"
    pool.prepare_lora_batch(["a"], weight_store=st)        # reload from the kept bank
    (again,) = st["a"].banks.values()
    assert again is bank
    s = pool.get_slot_id("a")
    for k in plan.keys:
        a_stack, b_stack = pool.get_module_buffers(k)
        assert torch.equal(a_stack[s, :4], a_mods[k][0]) and torch.equal(b_stack[s, :, :4], a_mods[k][1])
    # a pool that learned the same module keys from another adapter reuses the bank
    other = LoRAMemoryPool(2, 8, torch.device("cpu"), torch.float32)
    other.prepare_lora_batch(["d"], weight_store={"d": adapter(4, 4)})
    other.prepare_lora_batch(["a"], weight_store=st)
    assert next(iter(st["a"].banks.values())) is bank
    s = other.get_slot_id("a")
    assert torch.equal(other.get_module_buffers("v_proj")[1][s, :, :4], a_mods["v_proj"][1])


def test_new_module_keys_repack_or_raise_for_released_adapters():
    """A pool that grows a module key needs new banks: an adapter that still
    has its tensors is repacked; one whose tensors were released raises."""
    only_q = {"a": adapter(1, 2, keys=("q_proj",)), "b": adapter(2, 2, keys=("q_proj",))}
    both = {"c": adapter(3, 2)}
    pool = LoRAMemoryPool(2, 4, torch.device("cpu"), torch.float32)
    pool.buffers.release_modules = False
    pool.prepare_lora_batch(["a"], weight_store=only_q)
    pool.prepare_lora_batch(["c"], weight_store=both)      # adds v_proj
    pool.prepare_lora_batch(["b", "c"], weight_store={**only_q, **both})   # evicts "a"
    pool.prepare_lora_batch(["a", "c"], weight_store={**only_q, **both})   # repacked for q|v
    s = pool.get_slot_id("a")
    assert torch.equal(pool.get_module_buffers("q_proj")[0][s, :2], only_q["a"].modules["q_proj"][0])
    assert not pool.get_module_buffers("v_proj")[0][s].any()

    released = {"a": adapter(1, 2, keys=("q_proj",)), "b": adapter(2, 2, keys=("q_proj",))}
    pool = LoRAMemoryPool(2, 4, torch.device("cpu"), torch.float32)
    pool.prepare_lora_batch(["a"], weight_store=released)
    pool.prepare_lora_batch(["c"], weight_store=both)
    pool.prepare_lora_batch(["b", "c"], weight_store={**released, **both})
    with pytest.raises(RuntimeError, match="cannot be rebuilt"):
        pool.prepare_lora_batch(["a", "c"], weight_store={**released, **both})
