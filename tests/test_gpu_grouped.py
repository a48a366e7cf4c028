"""Slot-planned decode path (mlora_apply_grouped) against the oracle (GPU).

The decode path follows the table's plan (one entry per referenced slot and
up to 16 of its rows), reads each entry's A and B once per call, and in the
single launch hands K-chunk sums between work items of one XCD through its
L2.  Its arithmetic per row equals shrink-then-expand up to the order of
the fp32 K-reduction, so it is held to the float64 tolerance and to one
unit of the kernels' rounding sequence; its schedules (one launch, two
launches, and one launch whose waits all give up so that every expand item
computes every chunk itself) must agree bit for bit, and so must a plan
built on the host and one built on the device.
"""

import numpy as np
import pytest
import torch

from multi_lora_amd import HipLoRABackend, _ffi, synthetic
from multi_lora_amd.batch_info import (BatchLoRAInfo, build_plan, empty_kernel_input_metadata, plan_words,
                                       write_kernel_input_metadata)
from multi_lora_amd.kernels.lora_ops import LinkedWorkspace, apply_grouped, build_plan_device
from multi_lora_amd.synthetic import make_meta
from oracle.lora_ref import apply_f64, apply_kernel_numerics
from oracle.metadata_ref import plan_ref
from tests.gpu_helpers import assert_tol_f64, assert_ulp_close
from tests.test_gpu_lora import cpu_meta, run_hip

pytestmark = pytest.mark.gpu


def counters(lws: LinkedWorkspace):
    torch.cuda.synchronize()
    return lws.counters()


def assert_clean(lws: LinkedWorkspace):
    """No plan error; every chunk reached its consumers through the L2."""
    fb, pe = counters(lws)
    assert pe == 0, f"{pe} plan errors"
    assert fb == 0, f"{fb} chunks were computed after a wait gave up"


def grouped(wl, mode=0, lws=None, phases_split=False, meta=None):
    out = wl.clone_base()
    lws = lws if lws is not None else LinkedWorkspace()
    meta = wl.meta if meta is None else meta
    if phases_split:
        assert apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, meta, out, wl.col_offsets, lws, phases=1, mode=2)
        assert apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, meta, out, wl.col_offsets, lws, phases=2, mode=2)
    else:
        assert apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, meta, out, wl.col_offsets, lws, mode=mode)
    torch.cuda.synchronize()
    return out.cpu()


def check(wl, mode=0, lws=None):
    lws = lws if lws is not None else LinkedWorkspace()
    got = grouped(wl, mode, lws)
    cm = cpu_meta(wl.meta)
    xs, As, Bs, base = wl.x.cpu(), [a.cpu() for a in wl.a_stacks], [b.cpu() for b in wl.b_stacks], wl.base.cpu()
    assert_tol_f64(got, apply_f64(xs, As, Bs, cm, base, wl.col_offsets), f"{wl.name} vs float64")
    assert_ulp_close(got, apply_kernel_numerics(xs, As, Bs, cm, base, wl.col_offsets)[1], what=f"{wl.name}")
    _, pe = counters(lws)
    assert pe == 0
    return got


def workload(name, dev, lens, slots, ranks, scal, in_dim, outs, r_max, seed, dtype=torch.bfloat16, with_plan=True):
    g = torch.Generator().manual_seed(seed)
    n_slots = len(ranks)
    rows = sum(lens)
    x = torch.randn(rows, in_dim, generator=g).to(dtype)
    As = [(torch.randn(n_slots, r_max, in_dim, generator=g) * in_dim ** -0.5).to(dtype) for _ in outs]
    Bs = [(torch.randn(n_slots, o, r_max, generator=g) * 0.05).to(dtype) for o in outs]
    base = torch.randn(rows, sum(outs), generator=g).to(dtype)
    cols = [sum(outs[:i]) for i in range(len(outs))]
    meta = make_meta(lens, slots, ranks, scal, dev, dtype, with_plan=with_plan)
    return synthetic.LoRAWorkload(name, x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs], base.to(dev),
                                  meta, cols, lens, slots, ranks, scal)


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_decode_q_headline_shape(dev, mode):
    lws = LinkedWorkspace()
    check(synthetic.decode_q(device=dev), mode=mode, lws=lws)
    if mode != 2:
        assert_clean(lws)


def test_schedules_are_bit_identical(dev):
    """One launch, two launches, two launches run as separate halves, and one
    launch whose every wait gives up at once (each expand item computes all
    of its chunks itself) give the same bits."""
    wl = synthetic.decode_q(device=dev, tokens=128, seed=5)
    lws = LinkedWorkspace()
    one = grouped(wl, mode=1, lws=lws)
    assert_clean(lws)
    assert torch.equal(one, grouped(wl, mode=2))
    assert torch.equal(one, grouped(wl, phases_split=True))
    forced = LinkedWorkspace()
    grouped(wl, mode=1, lws=forced)  # allocate the buffer, then forbid waiting
    forced.set_wait_ticks(-1)
    assert torch.equal(one, grouped(wl, mode=1, lws=forced))
    fb, pe = counters(forced)
    assert fb > 0 and pe == 0


@pytest.mark.parametrize("outs,rank", [([1024, 256, 256], 16), ([768, 768], 32), ([512, 256, 256, 128], 16)])
def test_four_block_forced_fallback_equals_handoff(dev, outs, rank):
    """Four 16-row A blocks per shrink item with one expand K-step (q|k|v at
    rank 16, gate|up at rank 32, four slices at rank 16): the expand items'
    recompute of a missing chunk runs one A block at a time there, and must
    give the chunk sums the shrink items hand over, bit for bit."""
    g = torch.Generator().manual_seed(rank + len(outs))
    n_slots, rows = 24, 96
    slots = torch.randint(0, n_slots, (rows,), generator=g).tolist()
    ranks = [rank] * n_slots
    ranks[5] = 0
    wl = workload("four_blocks", dev, [1] * rows, slots, ranks, [1.5] * n_slots, 2048, outs, rank, 40 + rank)
    ref = check(wl, mode=1)
    lws = LinkedWorkspace()
    grouped(wl, mode=1, lws=lws)
    lws.set_wait_ticks(-1)
    assert torch.equal(grouped(wl, mode=1, lws=lws), ref)
    fb, pe = counters(lws)
    assert fb > 0 and pe == 0


@pytest.mark.parametrize("mode", [0, 2])
def test_decode_qkv_three_slices(dev, mode):
    check(synthetic.decode_qkv(device=dev), mode=mode)


def test_decode_qkv_forced_fallback_equals_handoff(dev):
    """Per-slice shrink items (three slices of rank 32): with every wait
    given up, the chunks each expand item computes equal what the shrink
    items hand over."""
    wl = synthetic.decode_qkv(device=dev, tokens=64)
    ref = grouped(wl, mode=1)
    lws = LinkedWorkspace()
    grouped(wl, mode=1, lws=lws)
    lws.set_wait_ticks(-1)
    assert torch.equal(grouped(wl, mode=1, lws=lws), ref)
    assert counters(lws)[0] > 0


@pytest.mark.parametrize("rank,r_max", [(64, 64), (40, 64), (8, 16), (13, 16)])
def test_ranks_and_partial_k_chunk(dev, rank, r_max):
    """Rank below r_max (stale tails), r_max 64, in_dim not a multiple of the
    256-wide K chunk, out not a multiple of the 256-column tile, a rank-0 slot."""
    g = torch.Generator().manual_seed(rank)
    n_slots, rows = 6, 40
    slots = torch.randint(0, n_slots, (rows,), generator=g).tolist()
    ranks = [rank] * n_slots
    ranks[2] = 0
    wl = workload("odd", dev, [1] * rows, slots, ranks, [1.5] * n_slots, 1000, [1288], r_max, rank)
    outs = {m: check(wl, mode=m) for m in (1, 2)}
    assert torch.equal(outs[1], outs[2])


@pytest.mark.parametrize("n_slots", [200, 300])
def test_live_slots_scattered_over_the_pool(dev, n_slots):
    """Live slots spread over a large pool; segments of rank-0, past-the-pool
    and negative slots keep the residual bit for bit."""
    g = torch.Generator().manual_seed(n_slots)
    live = [3, 64, 65, 127, 150, 199] + ([255, 256, 299] if n_slots > 256 else [])
    ranks = [0] * n_slots
    for i, s in enumerate(live):
        ranks[s] = 16 if i % 2 == 0 else 8
    rows = 72
    slots = [live[int(i)] for i in torch.randint(0, len(live), (rows,), generator=g)]
    slots[4], slots[9], slots[17] = 0, n_slots, -1
    scal = [0.5 + 0.01 * i for i in range(n_slots)]
    wl = workload("live_slots", dev, [1] * rows, slots, ranks, scal, 512, [768], 16, n_slots)
    for mode in (1, 2):
        got = check(wl, mode=mode)
        for r in (4, 9, 17):
            assert torch.equal(got[r], wl.base.cpu()[r])


def test_resident_adapters_the_batch_does_not_use(dev):
    """A steady-state pool: 64 resident rank-16 adapters, 128 decode tokens
    drawn over 32 of them.  Results match the oracle (the plan has entries
    for the 32 referenced slots only, so the others are never read)."""
    g = torch.Generator().manual_seed(77)
    n_slots, rows = 64, 128
    used = torch.randperm(n_slots, generator=g)[:32].tolist()
    slots = [used[int(i)] for i in torch.randint(0, 32, (rows,), generator=g)]
    wl = workload("resident64_used32", dev, [1] * rows, slots, [16] * n_slots, [2.0] * n_slots, 4096, [4096], 16, 78)
    assert wl.meta.plan_entries == len(set(slots))
    check(wl, mode=0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_grouped_matches_segment_kernels(dev, dtype):
    wl = synthetic.decode_q(device=dev, dtype=dtype, tokens=96, in_dim=2048, out=1536, n_slots=24, n_adapters=11,
                            rank=32, seed=9)
    got = grouped(wl)
    _, seg_out = run_hip(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, wl.base)
    assert_ulp_close(got, seg_out, what="grouped vs segment kernels")


def test_many_rows_per_slot_and_multi_row_segments(dev):
    """Slots with hundreds of rows (many 16-row entries each), segments of up
    to 16 rows, empty segments, rank-0 and foreign slots."""
    g = torch.Generator().manual_seed(31)
    lens = torch.randint(0, 17, (120,), generator=g).tolist()
    slots = torch.randint(0, 3, (120,), generator=g).tolist()
    slots[5], slots[6] = 9, -2
    ranks = [16, 0, 8]
    wl = workload("many_rows", dev, lens, slots, ranks, [2.0, 1.0, 0.5], 512, [768], 16, 31)
    assert wl.meta.plan_entries > 20
    got = check(wl)
    base = wl.base.cpu()
    st = 0
    for n, s in zip(lens, slots):
        if not (0 <= s < 3) or ranks[s] == 0:
            assert torch.equal(got[st:st + n], base[st:st + n])
        st += n


def test_host_and_device_plans_give_the_same_bits(dev):
    """A table without a plan gets one built on the device for the call."""
    wl = synthetic.decode_q(device=dev, tokens=100, in_dim=2048, out=1024, n_slots=40, n_adapters=23, rank=16, seed=8)
    bare = make_meta(wl.seg_lens, wl.seg_slots, wl.slot_ranks, wl.scalings, dev, torch.bfloat16, with_plan=False)
    assert bare.plan is None and wl.meta.plan is not None
    for mode in (1, 2):
        assert torch.equal(grouped(wl, mode=mode), grouped(wl, mode=mode, meta=bare))


def test_device_plan_kept_with_the_table_follows_in_place_rewrites(dev):
    """A table without a plan gets one built on the device once and kept
    while its tensors are unchanged; an in-place rewrite of a column (torch
    bumps its version) makes the next call build a new one.  Every call
    equals the same call with a host-built plan, bit for bit."""
    wl = synthetic.decode_q(device=dev, tokens=64, in_dim=1024, out=512, n_slots=16, n_adapters=9, rank=16, seed=83)
    bare = make_meta(wl.seg_lens, wl.seg_slots, wl.slot_ranks, wl.scalings, dev, torch.bfloat16,
                     host_copies=False, with_plan=False)
    lws = LinkedWorkspace()
    for mode in (1, 2):
        assert torch.equal(grouped(wl, mode=mode, lws=lws, meta=bare), grouped(wl, mode=mode))
    first = bare._device_plan
    assert torch.equal(grouped(wl, mode=1, lws=lws, meta=bare), grouped(wl, mode=1))
    assert bare._device_plan is first
    torch.cuda.synchronize()
    assert first.ready.query() and int(first.count_host[0]) == wl.meta.plan_entries
    # Rewrite the slots in place: rows move to other adapters.
    new_slots = [(s + 3) % 9 for s in wl.seg_slots]
    bare.weight_indices.copy_(torch.tensor(new_slots, dtype=torch.int32))
    moved = synthetic.LoRAWorkload(**{**wl.__dict__, "seg_slots": new_slots,
                                      "meta": make_meta(wl.seg_lens, new_slots, wl.slot_ranks, wl.scalings, dev,
                                                        torch.bfloat16)})
    got = grouped(wl, mode=1, lws=lws, meta=bare)
    assert bare._device_plan is not first
    assert torch.equal(got, grouped(moved, mode=1))
    assert counters(lws)[1] == 0


@pytest.mark.parametrize("seed", range(6))
def test_device_plan_builder_matches_host_and_oracle(dev, seed):
    g = torch.Generator().manual_seed(100 + seed)
    n_slots = [5, 64, 300, 2048, 17, 128][seed]
    bs = [0, 128, 200, 700, 40, 1500][seed]
    lens = torch.randint(0, 6 if seed % 2 else 17, (bs,), generator=g).tolist()
    slots = torch.randint(-2, n_slots + 2, (bs,), generator=g).tolist()
    ranks = [int(r) for r in torch.randint(0, 3, (n_slots,), generator=g) * 8]
    scal = [0.25 + 0.5 * (i % 7) for i in range(n_slots)]
    meta = make_meta(lens, slots, ranks, scal, dev, torch.bfloat16, with_plan=False)
    indptr = [0]
    for n in lens:
        indptr.append(indptr[-1] + n)
    rows = indptr[-1] - (3 if seed == 3 else 0)  # rows past the call are clamped away
    cap = max(1, rows)
    got = build_plan_device(meta, rows, n_slots, cap).cpu().numpy()
    host = np.zeros(plan_words(cap), dtype=np.int32)
    scal_f32 = torch.tensor(scal, dtype=torch.bfloat16).float().numpy()
    n = build_plan(indptr, slots, ranks, scal_f32, n_slots, rows, host)
    assert got[0] == n
    assert np.array_equal(got, host)
    ref = plan_ref(indptr, slots, ranks, scal_f32.view(np.int32).tolist(), n_slots, rows, cap)
    assert got.tolist() == ref


def test_workspace_reused_across_shapes(dev):
    """One workspace serves calls of different row counts, slot counts, slice
    counts and ranks in a row; each call matches the oracle although the
    flags and sums of the calls before it are still in the workspace."""
    lws = LinkedWorkspace()
    cases = [
        synthetic.decode_q(device=dev, tokens=128, seed=11),
        synthetic.decode_q(device=dev, tokens=24, in_dim=1024, out=768, n_slots=8, n_adapters=5, rank=32, seed=12),
        synthetic.decode_qkv(device=dev),
        synthetic.decode_q(device=dev, tokens=200, in_dim=2048, out=512, n_slots=40, n_adapters=30, rank=8, seed=13),
        synthetic.decode_q(device=dev, tokens=7, seed=14),
    ]
    for wl in cases:
        got = grouped(wl, mode=1, lws=lws)
        cm = cpu_meta(wl.meta)
        xs, As, Bs = wl.x.cpu(), [a.cpu() for a in wl.a_stacks], [b.cpu() for b in wl.b_stacks]
        assert_ulp_close(got, apply_kernel_numerics(xs, As, Bs, cm, wl.base.cpu(), wl.col_offsets)[1], what=wl.name)
    assert counters(lws)[1] == 0


def test_more_entries_than_grid_rows(dev):
    """A host entry count below the plan's (as in a graph captured on a
    smaller batch): workgroups loop over entries e, e + E, ... and the
    results stay the same."""
    wl = synthetic.decode_q(device=dev, tokens=128, in_dim=2048, out=2048, n_slots=64, n_adapters=40, rank=16, seed=15)
    ref = grouped(wl, mode=1)
    assert wl.meta.plan_entries > 24
    wl.meta.plan_entries = 1  # grid of 8 entry slots for the ~38 entries
    for mode in (1, 2):
        assert torch.equal(grouped(wl, mode=mode), ref)


def test_plan_too_small_is_reported(dev):
    """A plan with fewer entry slots than its table needs: the entries it
    holds are applied, the rest leave their rows untouched, and the
    workspace counts a plan error."""
    g = torch.Generator().manual_seed(16)
    rows = 24
    slots = list(range(rows))
    wl = workload("small_plan", dev, [1] * rows, slots, [16] * rows, [1.0] * rows, 256, [256], 16, 16)
    words = np.zeros(plan_words(4), dtype=np.int32)
    scal_f32 = torch.tensor(wl.scalings, dtype=torch.bfloat16).float().numpy()
    n = build_plan([i for i in range(rows + 1)], slots, wl.slot_ranks, scal_f32, rows, rows, words)
    assert n == rows
    wl.meta.plan, wl.meta.plan_cap, wl.meta.plan_entries = torch.from_numpy(words).to(dev), 4, n
    lws = LinkedWorkspace()
    got = grouped(wl, mode=1, lws=lws)
    assert counters(lws)[1] > 0
    base = wl.base.cpu()
    assert not torch.equal(got[:4], base[:4])
    assert torch.equal(got[4:], base[4:])


@pytest.mark.parametrize("mode", [1, 2])
def test_plan_for_more_rows_than_the_call(dev, mode):
    """A plan made for a longer table than the call (40 rows planned, 24
    rows called): plan rows at or past the call's rows are not stored, and
    no row receives another row's delta.  Every output row is either left
    untouched or equal, bit for bit, to the same call with a table of the
    24 rows; some rows are computed, and the workspace counts plan errors."""
    wl = synthetic.decode_q(device=dev, tokens=40, in_dim=1024, out=512, n_slots=8, n_adapters=5, rank=16, seed=81)
    rows = 24
    x, base = wl.x[:rows], wl.base[:rows]
    lws = LinkedWorkspace()
    out = base.clone()
    assert apply_grouped(x, wl.a_stacks, wl.b_stacks, wl.meta, out, [0], lws, mode=mode)
    proper = make_meta(wl.seg_lens[:rows], wl.seg_slots[:rows], wl.slot_ranks, wl.scalings, dev, torch.bfloat16)
    want = base.clone()
    assert apply_grouped(x, wl.a_stacks, wl.b_stacks, proper, want, [0], LinkedWorkspace(), mode=mode)
    assert counters(lws)[1] > 0
    got, want, base = out.cpu(), want.cpu(), base.cpu()
    untouched = (got == base).all(dim=1)
    computed = (got == want).all(dim=1)
    assert bool((untouched | computed).all())
    assert bool((computed & ~(want == base).all(dim=1)).any())


def test_device_plan_into_a_dirty_buffer(dev):
    """mlora_build_plan writes every header word (the rest 0) and every word of
    the entries it makes, so a buffer full of garbage gives the host's plan."""
    wl = synthetic.decode_q(device=dev, tokens=50, in_dim=1024, out=512, n_slots=12, n_adapters=7, rank=16, seed=82)
    cap = 50
    bare = make_meta(wl.seg_lens, wl.seg_slots, wl.slot_ranks, wl.scalings, dev, torch.bfloat16, with_plan=False)
    lib = _ffi.lib()
    words = lib.mlora_plan_bytes(cap) // 4
    plan = torch.full((words,), -123457, dtype=torch.int32, device=dev)
    from multi_lora_amd.kernels.lora_ops import seg_meta
    import ctypes
    m, keep = seg_meta(bare, dev, 12)
    m.plan, m.plan_cap, m.plan_entries = None, 0, -1
    _ffi.check(lib.mlora_build_plan(ctypes.byref(m), 50, plan.data_ptr(), cap, _ffi.stream_ptr(dev)), "build_plan")
    torch.cuda.synchronize()
    got = plan.cpu().numpy()
    host = np.zeros(plan_words(cap), dtype=np.int32)
    indptr = [0]
    for n in wl.seg_lens:
        indptr.append(indptr[-1] + n)
    scal_f32 = torch.tensor(wl.scalings, dtype=torch.bfloat16).float().numpy()
    n = build_plan(indptr, wl.seg_slots, wl.slot_ranks, scal_f32, 12, 50, host)
    used = 16 + n * 32
    assert np.array_equal(got[:used], host[:used])
    del keep


def test_linked_repeated_calls_are_bit_identical(dev):
    wl = synthetic.decode_q(device=dev, tokens=128, seed=21)
    lws = LinkedWorkspace()
    first = grouped(wl, mode=1, lws=lws)
    for _ in range(5):
        assert torch.equal(grouped(wl, mode=1, lws=lws), first)
    assert_clean(lws)


def test_linked_same_shape_new_inputs_each_call(dev):
    """Calls of one shape in a row with new inputs: every flag still holds
    the previous call's tag when the next call starts, and must not be taken
    for the new one."""
    lws = LinkedWorkspace()
    for seed in range(30, 36):
        wl = synthetic.decode_q(device=dev, tokens=128, seed=seed)
        got = grouped(wl, mode=1, lws=lws)
        cm = cpu_meta(wl.meta)
        ref = apply_kernel_numerics(wl.x.cpu(), [wl.a_stacks[0].cpu()], [wl.b_stacks[0].cpu()], cm, wl.base.cpu())[1]
        assert_ulp_close(got, ref, what=f"seed {seed}")
    assert_clean(lws)


def test_workspace_keeps_streams_apart(dev):
    """One LinkedWorkspace used from two streams holds one buffer per stream."""
    lws = LinkedWorkspace()
    wl = synthetic.decode_q(device=dev, tokens=64, seed=41)
    ref = grouped(wl, mode=1, lws=lws)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        out = wl.clone_base()
        assert apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, out, wl.col_offsets, lws, mode=1)
    torch.cuda.synchronize()
    assert len(lws.bufs) == 2
    assert torch.equal(out.cpu(), ref)
    assert_clean(lws)


def test_ineligible_shapes_fall_back(dev):
    wl = synthetic.decode_q(device=dev, dtype=torch.float32, tokens=8, in_dim=256, out=256, n_slots=4, n_adapters=2,
                            rank=16)
    out = wl.clone_base()
    assert not apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, out, [0])
    be = HipLoRABackend()
    be.set_kernel_input_metadata(wl.meta)
    got = be.apply_lora(wl.x, wl.a_stacks[0], wl.b_stacks[0], wl.clone_base())
    assert_tol_f64(got.cpu(), apply_f64(wl.x.cpu(), [wl.a_stacks[0].cpu()], [wl.b_stacks[0].cpu()],
                                        cpu_meta(wl.meta), wl.base.cpu()))


def test_backend_uses_grouped_for_decode_and_is_deterministic(dev):
    wl = synthetic.decode_q(device=dev, tokens=128, seed=2)
    be = HipLoRABackend()
    be.set_kernel_input_metadata(wl.meta)
    outs = [be.apply_lora(wl.x, wl.a_stacks[0], wl.b_stacks[0], wl.clone_base()) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    assert torch.equal(outs[0].cpu(), grouped(wl))
    assert_clean(be.linked_workspace)


def _packed_meta(dev, slots, ranks, scal):
    info = BatchLoRAInfo(weight_indices=slots, lora_ranks=ranks, scalings=scal)
    return write_kernel_input_metadata(empty_kernel_input_metadata(device=dev, dtype=torch.bfloat16), info,
                                       device=dev, dtype=torch.bfloat16, seq_lens=[])


@pytest.mark.parametrize("plan", ["packed", "device"])
def test_hip_graph_replays_follow_metadata_rewrites(dev, plan):
    """A captured call replays correctly, and a segment table rewritten in
    place between replays takes effect: through write_kernel_input_metadata
    (which rebuilds the packed plan), or, for a table without a plan, through
    the device plan build captured with the call."""
    from multi_lora_amd.batch_info import fill_column

    wl = synthetic.decode_q(device=dev, tokens=64, in_dim=2048, out=2048, n_slots=16, n_adapters=8, rank=16, seed=3)
    a, b = wl.a_stacks[0], wl.b_stacks[0]
    if plan == "packed":
        meta = _packed_meta(dev, wl.seg_slots, wl.slot_ranks, wl.scalings)
        assert meta.plan is not None
    else:
        meta = make_meta(wl.seg_lens, wl.seg_slots, wl.slot_ranks, wl.scalings, dev, torch.bfloat16, with_plan=False)
    be = HipLoRABackend()
    be.set_kernel_input_metadata(meta)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # the capture stream's workspace exists before capture
        eager = be.apply_lora(wl.x, a, b, wl.clone_base())
    torch.cuda.synchronize()

    out = wl.clone_base()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        be.apply_lora(wl.x, a, b, out)
    for _ in range(4):
        out.copy_(wl.base)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)

    new_slots = [(s + 3) % 8 for s in wl.seg_slots]
    if plan == "packed":
        again = _packed_meta(dev, new_slots, wl.slot_ranks, wl.scalings)  # a reference for the new table
        assert write_kernel_input_metadata(
            meta, BatchLoRAInfo(new_slots, wl.slot_ranks, wl.scalings), device=dev, dtype=torch.bfloat16,
            seq_lens=[]) is meta
        ref_meta = again
    else:
        fill_column(meta.weight_indices, new_slots, 0)
        ref_meta = make_meta(wl.seg_lens, new_slots, wl.slot_ranks, wl.scalings, dev, torch.bfloat16)
    be2 = HipLoRABackend()
    be2.set_kernel_input_metadata(ref_meta)
    eager2 = be2.apply_lora(wl.x, a, b, wl.clone_base())
    torch.cuda.synchronize()
    assert not torch.equal(eager2, eager)
    for _ in range(3):
        out.copy_(wl.base)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager2)
    assert counters(be.linked_workspace)[1] == 0


@pytest.mark.parametrize("mode", [1, 2])
def test_slices_not_multiples_of_the_expand_tile(dev, mode):
    """Three slices of 520, 264 and 1000 columns packed into one output row:
    expand items straddle no slice boundary and write nothing past a slice's width."""
    g = torch.Generator().manual_seed(11 + mode)
    n_slots, rows = 9, 48
    slots = torch.randint(0, n_slots, (rows,), generator=g).tolist()
    ranks = [32, 17, 0, 32, 8, 32, 25, 32, 32]
    wl = workload("slices", dev, [1] * rows, slots, ranks, [1.25] * n_slots, 512, [520, 264, 1000], 32, 11 + mode)
    got = check(wl, mode=mode)
    for t, s in enumerate(slots):
        if ranks[s] == 0:
            assert torch.equal(got[t], wl.base.cpu()[t])


def test_abi_version(dev):
    assert _ffi.lib().mlora_abi_version() == _ffi.ABI_VERSION == 6


def test_largest_supported_shape(dev):
    """The decode path's limits together: in_dim 16384 (64 K chunks, one flag
    per lane of the polling wave), four slices at r_max 64 (shrink items split
    per slice), full and partial ranks, a rank-0 slot, segments of up to 16
    rows.  All schedules, and the single launch with every wait given up,
    agree bit for bit and match the oracle."""
    assert _ffi.lib().mlora_grouped_workspace_bytes(16384, 64, 4, 64, 8, _ffi.MLORA_BF16, 0) > 0
    g = torch.Generator().manual_seed(77)
    n_slots = 8
    lens = [1, 16, 3, 1, 7, 1, 1, 16, 2, 1, 1, 1, 5, 1, 1, 1]
    slots = torch.randint(0, n_slots, (len(lens),), generator=g).tolist()
    ranks = [64, 40, 0, 64, 17, 64, 64, 33]
    wl = workload("largest", dev, lens, slots, ranks, [0.75] * n_slots, 16384, [512, 256, 264, 1024], 64, 77)
    lws = LinkedWorkspace()
    one = check(wl, mode=1, lws=lws)
    assert_clean(lws)
    assert torch.equal(grouped(wl, mode=2), one)
    lws.set_wait_ticks(-1)
    assert torch.equal(grouped(wl, mode=1, lws=lws), one)
    assert counters(lws)[0] > 0
