"""Slot-grouped decode path (mlora_apply_grouped) against the oracle (GPU).

The grouped path reads each referenced adapter once per call and finds the
rows of every slot with an in-kernel scan of the segment table; its
arithmetic per row equals shrink-then-expand up to the order of the fp32
K-reduction, so it is held to the float64 tolerance and to one unit of the
kernels' rounding sequence.  The single-launch mode links its shrink and
expand work items through words tagged per launch: calls in a row on one
workspace, of any shapes, must each match the oracle, with the workspace's
error word still zero.
"""

import pytest
import torch

from multi_lora_amd import HipLoRABackend, synthetic
from multi_lora_amd.kernels.lora_ops import LinkedWorkspace, Workspace, apply_grouped
from multi_lora_amd.synthetic import make_meta
from oracle.lora_ref import apply_f64, apply_kernel_numerics
from oracle.metadata_ref import slot_gather_order
from tests.gpu_helpers import assert_tol_f64, assert_ulp_close
from tests.test_gpu_lora import cpu_meta, run_hip

pytestmark = pytest.mark.gpu


def assert_linked_clean(lws: LinkedWorkspace):
    """No wait between linked work items timed out."""
    torch.cuda.synchronize()
    assert lws.error_word() == 0, "a wait between linked work items timed out"


def grouped(wl, phases_split=False, mode=0, lws=None):
    out = wl.clone_base()
    ws = Workspace()
    lws = lws if lws is not None else LinkedWorkspace()
    if phases_split:
        assert apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, out, wl.col_offsets, ws, phases=1, mode=2)
        assert apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, out, wl.col_offsets, ws, phases=2, mode=2)
    else:
        assert apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, out, wl.col_offsets, ws, mode=mode,
                             linked_workspace=lws)
    torch.cuda.synchronize()
    if mode != 2 and not phases_split:
        assert_linked_clean(lws)
    return out.cpu()


def check(wl, phases_split=False, mode=0):
    got = grouped(wl, phases_split, mode)
    cm = cpu_meta(wl.meta)
    xs, As, Bs, base = wl.x.cpu(), [a.cpu() for a in wl.a_stacks], [b.cpu() for b in wl.b_stacks], wl.base.cpu()
    assert_tol_f64(got, apply_f64(xs, As, Bs, cm, base, wl.col_offsets), f"{wl.name} vs float64")
    assert_ulp_close(got, apply_kernel_numerics(xs, As, Bs, cm, base, wl.col_offsets)[1], what=f"{wl.name}")
    return got


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_decode_q_headline_shape(dev, mode):
    check(synthetic.decode_q(device=dev), mode=mode)


def test_decode_q_phases_split_equals_two_launch_call(dev):
    wl = synthetic.decode_q(device=dev, tokens=64, seed=7)
    assert torch.equal(grouped(wl, mode=2), grouped(wl, phases_split=True))


def test_single_and_two_launch_paths_agree(dev):
    wl = synthetic.decode_q(device=dev, tokens=128, seed=5)
    assert_ulp_close(grouped(wl, mode=1), grouped(wl, mode=2), what="single vs two launches")


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_decode_qkv_three_slices(dev, mode):
    check(synthetic.decode_qkv(device=dev), mode=mode)


@pytest.mark.parametrize("rank,r_max", [(64, 64), (40, 64), (8, 16)])
def test_single_launch_ranks_and_odd_k(dev, rank, r_max):
    """Rank below r_max (stale tails), r_max 64, in_dim not a multiple of 32, out not a multiple of 512."""
    g = torch.Generator().manual_seed(rank)
    n_slots, rows, in_dim, out_dim = 6, 40, 1000, 1288
    slots = torch.randint(0, n_slots, (rows,), generator=g).tolist()
    ranks = [rank] * n_slots
    ranks[2] = 0
    x = torch.randn(rows, in_dim, generator=g).bfloat16()
    a = (torch.randn(n_slots, r_max, in_dim, generator=g) * in_dim ** -0.5).bfloat16()
    b = (torch.randn(n_slots, out_dim, r_max, generator=g) * 0.05).bfloat16()
    base = torch.randn(rows, out_dim, generator=g).bfloat16()
    meta = make_meta([1] * rows, slots, ranks, [1.5] * n_slots, dev, torch.bfloat16)
    wl = synthetic.LoRAWorkload("odd", x.to(dev), [a.to(dev)], [b.to(dev)], base.to(dev), meta, [0], [1] * rows,
                                slots, ranks, [1.5] * n_slots)
    for mode in (1, 2):
        check(wl, mode=mode)


@pytest.mark.parametrize("n_slots", [200, 300])
def test_live_slots_scattered_over_the_pool(dev, n_slots):
    """Work items are numbered over the slots with a non-zero rank.  Live
    slots spread over several 64-slot chunks of the rank table (200 slots),
    and a pool too large for that numbering (300: numbered by slot); segments
    of rank-0 and out-of-pool slots keep the residual bit for bit."""
    g = torch.Generator().manual_seed(n_slots)
    live = [3, 64, 65, 127, 150, 199] + ([255, 256, 299] if n_slots > 256 else [])
    ranks = [0] * n_slots
    for i, s in enumerate(live):
        ranks[s] = 16 if i % 2 == 0 else 8
    rows, in_dim, out_dim = 72, 512, 768
    slots = [live[int(i)] for i in torch.randint(0, len(live), (rows,), generator=g)]
    slots[4], slots[9], slots[17] = 0, n_slots, -1  # rank 0, past the pool, negative
    x = torch.randn(rows, in_dim, generator=g).bfloat16()
    a = (torch.randn(n_slots, 16, in_dim, generator=g) * in_dim ** -0.5).bfloat16()
    b = (torch.randn(n_slots, out_dim, 16, generator=g) * 0.05).bfloat16()
    base = torch.randn(rows, out_dim, generator=g).bfloat16()
    scal = [0.5 + 0.01 * i for i in range(n_slots)]
    meta = make_meta([1] * rows, slots, ranks, scal, dev, torch.bfloat16)
    wl = synthetic.LoRAWorkload("live_slots", x.to(dev), [a.to(dev)], [b.to(dev)], base.to(dev), meta, [0],
                                [1] * rows, slots, ranks, scal)
    for mode in (1, 2):
        got = check(wl, mode=mode)
        for r in (4, 9, 17):
            assert torch.equal(got[r], base[r])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_grouped_matches_segment_kernels(dev, dtype):
    wl = synthetic.decode_q(device=dev, dtype=dtype, tokens=96, in_dim=2048, out=1536, n_slots=24, n_adapters=11,
                            rank=32, seed=9)
    got = grouped(wl)
    _, seg_out = run_hip(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, wl.base)
    assert_ulp_close(got, seg_out, what="grouped vs segment kernels")


def test_many_rows_per_slot_and_multi_row_segments(dev):
    """More than one 256-row window for a slot, segments of up to 16 rows, rank-0 and foreign slots."""
    g = torch.Generator().manual_seed(31)
    lens = torch.randint(0, 17, (120,), generator=g).tolist()
    slots = torch.randint(0, 3, (120,), generator=g).tolist()
    slots[5], slots[6] = 9, -2  # outside the pool: untouched rows
    ranks = [16, 0, 8]
    in_dim, out_dim = 512, 768
    rows = sum(lens)
    x = torch.randn(rows, in_dim, generator=g).bfloat16()
    a = (torch.randn(3, 16, in_dim, generator=g) * in_dim ** -0.5).bfloat16()
    b = (torch.randn(3, out_dim, 16, generator=g) * 0.05).bfloat16()
    base = torch.randn(rows, out_dim, generator=g).bfloat16()
    indptr = [0]
    for n in lens:
        indptr.append(indptr[-1] + n)
    _, offs, _ = slot_gather_order(indptr, slots, ranks, len(lens))
    assert max(offs[i + 1] - offs[i] for i in range(len(offs) - 1)) > 256
    meta = make_meta(lens, slots, ranks, [2.0, 1.0, 0.5], dev, torch.bfloat16)
    wl = synthetic.LoRAWorkload("many_rows", x.to(dev), [a.to(dev)], [b.to(dev)], base.to(dev), meta, [0], lens,
                                slots, ranks, [2.0, 1.0, 0.5])
    got = check(wl)
    # rows of rank-0 or out-of-pool segments are bit-identical to the residual
    st = 0
    for n, s in zip(lens, slots):
        if not (0 <= s < 3) or ranks[s] == 0:
            assert torch.equal(got[st:st + n], base[st:st + n])
        st += n


def test_linked_workspace_reused_across_shapes(dev):
    """One single-launch workspace serves calls of different row counts, slot
    counts, slice counts and ranks in a row; each call matches the oracle
    although the words of the calls before it are still in the workspace."""
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


def test_auto_mode_switches_schedules_on_one_workspace(dev):
    """Mode 0 takes the single launch for small batches and two launches for
    large ones (fp32 sums in the region after the tagged words); alternating between
    them, with shapes changing, every call still matches the oracle."""
    from multi_lora_amd import _ffi

    lws = LinkedWorkspace()
    small = synthetic.decode_q(device=dev, tokens=64, seed=51)
    large = synthetic.decode_qkv(device=dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    n_large = large.a_stacks[0].shape[0] * (3 * 16 + 16 + 4 + 4)   # slots x (shrink + expand items)
    assert n_large > 16 * cus, "the large case must exceed the single-launch limit"
    for wl in (small, large, small, large, small):
        got = grouped(wl, mode=0, lws=lws)
        cm = cpu_meta(wl.meta)
        xs, As, Bs = wl.x.cpu(), [a.cpu() for a in wl.a_stacks], [b.cpu() for b in wl.b_stacks]
        assert_ulp_close(got, apply_kernel_numerics(xs, As, Bs, cm, wl.base.cpu(), wl.col_offsets)[1], what=wl.name)
    assert _ffi.lib().mlora_abi_version() == _ffi.ABI_VERSION


def test_linked_repeated_calls_are_bit_identical(dev):
    wl = synthetic.decode_q(device=dev, tokens=128, seed=21)
    lws = LinkedWorkspace()
    first = grouped(wl, mode=1, lws=lws)
    for _ in range(5):
        assert torch.equal(grouped(wl, mode=1, lws=lws), first)


def test_linked_same_shape_new_inputs_each_call(dev):
    """Calls of one shape in a row with new inputs: every word position still
    holds the previous call's sum when the next call starts, and must not be
    taken for the new one."""
    lws = LinkedWorkspace()
    for seed in range(30, 36):
        wl = synthetic.decode_q(device=dev, tokens=128, seed=seed)
        got = grouped(wl, mode=1, lws=lws)
        cm = cpu_meta(wl.meta)
        ref = apply_kernel_numerics(wl.x.cpu(), [wl.a_stacks[0].cpu()], [wl.b_stacks[0].cpu()], cm, wl.base.cpu())[1]
        assert_ulp_close(got, ref, what=f"seed {seed}")


def test_linked_workspace_keeps_streams_apart(dev):
    """One LinkedWorkspace used from two streams holds one buffer per stream."""
    lws = LinkedWorkspace()
    wl = synthetic.decode_q(device=dev, tokens=64, seed=41)
    ref = grouped(wl, mode=1, lws=lws)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        out = wl.clone_base()
        assert apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, out, wl.col_offsets, mode=1,
                             linked_workspace=lws)
    torch.cuda.synchronize()
    assert len(lws.bufs) == 2
    assert torch.equal(out.cpu(), ref)
    assert_linked_clean(lws)


def test_ineligible_shapes_fall_back(dev):
    wl = synthetic.decode_q(device=dev, dtype=torch.float32, tokens=8, in_dim=256, out=256, n_slots=4, n_adapters=2,
                            rank=16)
    out = wl.clone_base()
    assert not apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, out, [0])
    # the backend then takes the segment kernels and still matches
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


def test_hip_graph_replays_match_eager_and_follow_metadata_rewrites(dev):
    """Kernels read every per-step value from device memory: a captured call
    replays correctly, and rewriting the segment table in place between
    replays (as write_kernel_input_metadata does) takes effect."""
    from multi_lora_amd.batch_info import fill_column

    wl = synthetic.decode_q(device=dev, tokens=64, in_dim=2048, out=2048, n_slots=16, n_adapters=8, rank=16, seed=3)
    a, b = wl.a_stacks[0], wl.b_stacks[0]
    be = HipLoRABackend()
    be.set_kernel_input_metadata(wl.meta)
    eager = be.apply_lora(wl.x, a, b, wl.clone_base())
    torch.cuda.synchronize()

    out = wl.clone_base()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        be.apply_lora(wl.x, a, b, out)
    for _ in range(4):
        out.copy_(wl.base)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert_linked_clean(be.linked_workspace)

    # New slot assignment, written in place into the captured table.
    new_slots = [(s + 3) % 8 for s in wl.seg_slots]
    fill_column(wl.meta.weight_indices, new_slots, 0)
    be2 = HipLoRABackend()
    be2.set_kernel_input_metadata(wl.meta)
    eager2 = be2.apply_lora(wl.x, a, b, wl.clone_base())
    torch.cuda.synchronize()
    assert not torch.equal(eager2, eager)
    for _ in range(3):
        out.copy_(wl.base)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager2)
    assert_linked_clean(be.linked_workspace)


@pytest.mark.parametrize("mode", [1, 2])
def test_slices_not_multiples_of_the_expand_tile(dev, mode):
    """Three slices of 520, 264 and 1000 columns packed into one output row:
    expand items (256 columns in the single launch, 512 with two launches)
    straddle no slice boundary and write nothing past a slice's width."""
    g = torch.Generator().manual_seed(11 + mode)
    n_slots, rows, in_dim, r_max = 9, 48, 512, 32
    outs = [520, 264, 1000]
    slots = torch.randint(0, n_slots, (rows,), generator=g).tolist()
    ranks = [32, 17, 0, 32, 8, 32, 25, 32, 32]
    x = torch.randn(rows, in_dim, generator=g).bfloat16()
    As = [(torch.randn(n_slots, r_max, in_dim, generator=g) * in_dim ** -0.5).bfloat16() for _ in outs]
    Bs = [(torch.randn(n_slots, o, r_max, generator=g) * 0.05).bfloat16() for o in outs]
    base = torch.randn(rows, sum(outs), generator=g).bfloat16()
    cols = [0, outs[0], outs[0] + outs[1]]
    meta = make_meta([1] * rows, slots, ranks, [1.25] * n_slots, dev, torch.bfloat16)
    wl = synthetic.LoRAWorkload("slices", x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs], base.to(dev),
                                meta, cols, [1] * rows, slots, ranks, [1.25] * n_slots)
    got = check(wl, mode=mode)
    for t, s in enumerate(slots):
        if ranks[s] == 0:
            assert torch.equal(got[t], base[t])
