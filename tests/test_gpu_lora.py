"""HIP shrink/expand parity against the oracle (GPU).

Every case runs the library's kernels through the C ABI (via the
``sgemm_lora_*`` entry points) on seeded inputs and compares with
* the float64 closed form (``apply_f64``) at the path's tolerance, and
* the oracle's restatement of the kernels' rounding sequence
  (``apply_kernel_numerics``) to within one unit in the last place.
"""

import pytest
import torch

from multi_lora_amd import synthetic
from multi_lora_amd.kernels import (
    sgemm_lora_a_fwd,
    sgemm_lora_a_multi_fwd,
    sgemm_lora_b_fwd,
    sgemm_lora_b_multi_fwd,
)
from multi_lora_amd.kernels.lora_ops import Workspace, apply_segments, shrink
from multi_lora_amd.synthetic import make_meta
from oracle.lora_ref import TorchLoRABackend, apply_f64, apply_kernel_numerics
from tests.gpu_helpers import assert_tol_f64, assert_ulp_close

pytestmark = pytest.mark.gpu


def run_hip(x, a_stacks, b_stacks, meta, base, cols=None):
    """Shrink then expand on the GPU; returns (mid, out) on the CPU."""
    r_max = a_stacks[0].shape[1]
    mid = torch.full((x.shape[0], len(a_stacks) * r_max), float("nan"), dtype=x.dtype, device=x.device)
    out = base.clone()
    if len(a_stacks) == 1:
        sgemm_lora_a_fwd(x, a_stacks[0], meta, mid)
        sgemm_lora_b_fwd(mid, b_stacks[0], meta, base_output=out)
    else:
        sgemm_lora_a_multi_fwd(x, a_stacks, meta, mid)
        sgemm_lora_b_multi_fwd(mid, b_stacks, meta, out, cols)
    torch.cuda.synchronize()
    return mid.cpu(), out.cpu()


def cpu_meta(meta):
    return type(meta)(
        bs=meta.bs, seg_lens=meta.seg_lens.cpu(), seg_indptr=meta.seg_indptr.cpu(),
        weight_indices=meta.weight_indices.cpu(), lora_ranks=meta.lora_ranks.cpu(),
        scalings=meta.scalings.cpu(), max_len=meta.max_len)


def check_workload(wl, tight=True):
    cols = wl.col_offsets
    mid, out = run_hip(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, wl.base, cols)
    cm = cpu_meta(wl.meta)
    xs, As, Bs, base = wl.x.cpu(), [a.cpu() for a in wl.a_stacks], [b.cpu() for b in wl.b_stacks], wl.base.cpu()
    want64 = apply_f64(xs, As, Bs, cm, base, cols)
    assert_tol_f64(out, want64, f"{wl.name} vs float64")
    if tight:
        kmid, kout = apply_kernel_numerics(xs, As, Bs, cm, base, cols)
        valid = torch.zeros(mid.shape[0], dtype=torch.bool)
        for s, n in enumerate(wl.seg_lens):
            st = sum(wl.seg_lens[:s])
            valid[st:st + n] = True
        assert_ulp_close(mid[valid], kmid[valid], what=f"{wl.name} mid")
        assert_ulp_close(out, kout, what=f"{wl.name} out")
    return mid, out


def test_decode_q_llama8b_shape(dev):
    """Decode q_proj 4096->4096 bf16, 128 single-token segments, 32 of 64 slots at rank 16."""
    check_workload(synthetic.decode_q(device=dev))


def test_cpu_small_config_in_fp32_on_gpu(dev):
    """The fp32 1024->1024 case: segments [5,17,42] -> slots [2,0,3], rank 8."""
    wl = synthetic.cpu_small(device=dev)
    mid, out = check_workload(wl)
    # also equal (to fp32 rounding) to the reference's per-segment PyTorch path
    be = TorchLoRABackend()
    be.set_kernel_input_metadata(cpu_meta(wl.meta))
    ref = be.apply_lora(wl.x.cpu(), wl.a_stacks[0].cpu(), wl.b_stacks[0].cpu(), wl.base.cpu().clone())
    torch.testing.assert_close(out, ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_decode_q_dtypes_small(dev, dtype):
    check_workload(synthetic.decode_q(device=dev, dtype=dtype, tokens=40, in_dim=512, out=768, n_slots=8,
                                      n_adapters=5, rank=16, seed=11))


def test_decode_qkv_multi_slice(dev):
    """Fused q|k|v [4096,1024,1024], 256 tokens over 128 rank-32 adapters in a 256-slot pool."""
    check_workload(synthetic.decode_qkv(device=dev))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_gate_up_reduced(dev, dtype):
    wl = synthetic.prefill_mlp(device=dev, dtype=dtype, part="gate_up", n_seg=4, min_len=17, max_len=200,
                               hidden=1024, inter=2816, seed=21)
    check_workload(wl)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_down_reduced(dev, dtype):
    wl = synthetic.prefill_mlp(device=dev, dtype=dtype, part="down", n_seg=5, min_len=1, max_len=150, hidden=768,
                               inter=3584, seed=22)
    check_workload(wl)


@pytest.mark.parametrize("part", ["gate_up", "down"])
def test_prefill_full_size_sampled_rows(dev, part):
    """Full prefill MLP shapes (~4k tokens); a sample of rows checked against float64."""
    wl = synthetic.prefill_mlp(device=dev, part=part)
    mid, out = run_hip(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, wl.base, wl.col_offsets)
    g = torch.Generator().manual_seed(0)
    rows = torch.randint(0, wl.tokens, (48,), generator=g).tolist()
    starts = [sum(wl.seg_lens[:i]) for i in range(len(wl.seg_lens))]
    x, base = wl.x.cpu().double(), wl.base.cpu().double()
    for t in rows:
        seg = max(i for i, s in enumerate(starts) if s <= t)
        slot = wl.seg_slots[seg]
        r = wl.slot_ranks[slot]
        want = base[t].clone()
        for a, b, c0 in zip(wl.a_stacks, wl.b_stacks, wl.col_offsets):
            y = x[t] @ a[slot, :r].cpu().double().T
            want[c0:c0 + b.shape[1]] += 2.0 * (y @ b[slot, :, :r].cpu().double().T)
        torch.testing.assert_close(out[t].double(), want, atol=2e-2, rtol=1e-2, msg=f"row {t}")


@pytest.mark.parametrize("rows_per_adapter", [2, 8])
def test_grouped_matches_rowwise_decode(dev, rows_per_adapter):
    """multi_lora/tests/test_grouped_rows.py:92-134 on the HIP kernels."""
    dt = torch.bfloat16
    torch.manual_seed(0)
    in_dim, out_dim, max_rank = 96, 256, 64
    ranks, scalings = [8, 16], [1.0, 2.0]
    a_stack = (torch.randn(2, max_rank, in_dim) * 0.1).to(dev, dt)
    b_stack = (torch.randn(2, out_dim, max_rank) * 0.1).to(dev, dt)
    rows = rows_per_adapter * 2
    x = torch.randn(rows, in_dim).to(dev, dt)
    widx_rows = [0] * rows_per_adapter + [1] * rows_per_adapter
    base = torch.randn(rows, out_dim).to(dev, dt)
    meta_group = make_meta([rows_per_adapter] * 2, [0, 1], ranks, scalings, dev, torch.float32)
    meta_row = make_meta([1] * rows, widx_rows, ranks, scalings, dev, torch.float32)
    assert meta_group.max_len > 1 and meta_row.max_len == 1
    outs = {}
    for tag, meta in (("group", meta_group), ("row", meta_row)):
        mid = torch.zeros(rows, max_rank, device=dev, dtype=dt)
        mid = sgemm_lora_a_fwd(x, a_stack, meta, mid)
        y = sgemm_lora_b_fwd(mid, b_stack, meta, base_output=base.clone())
        outs[tag] = (mid, y)
    for tag in ("group", "row"):
        mid = outs[tag][0]
        for row, slot in enumerate(widx_rows):
            assert (mid[row, ranks[slot]:] == 0).all(), (tag, row)
    ref = apply_f64(x.cpu(), [a_stack.cpu()], [b_stack.cpu()], cpu_meta(meta_row), base.cpu())
    torch.testing.assert_close(outs["group"][1].cpu(), outs["row"][1].cpu(), rtol=2e-2, atol=2e-2)
    assert_tol_f64(outs["group"][1].cpu(), ref)
    assert_tol_f64(outs["row"][1].cpu(), ref)
    # grouping changes only the tiling, never the per-row arithmetic
    assert torch.equal(outs["group"][1], outs["row"][1])


def test_grouped_matches_rowwise_prefill(dev):
    """multi_lora/tests/test_grouped_rows.py:137-165 on the HIP kernels."""
    dt = torch.bfloat16
    torch.manual_seed(1)
    in_dim, out_dim, max_rank = 96, 256, 64
    ranks, scalings = [8, 16], [1.0, 2.0]
    a_stack = (torch.randn(2, max_rank, in_dim) * 0.1).to(dev, dt)
    b_stack = (torch.randn(2, out_dim, max_rank) * 0.1).to(dev, dt)
    row_lens = [5, 5, 3, 3]
    total = sum(row_lens)
    x = torch.randn(total, in_dim).to(dev, dt)
    base = torch.randn(total, out_dim).to(dev, dt)
    meta_group = make_meta([10, 6], [0, 1], ranks, scalings, dev, torch.float32)
    meta_row = make_meta(row_lens, [0, 0, 1, 1], ranks, scalings, dev, torch.float32)
    outs = {}
    for tag, meta in (("group", meta_group), ("row", meta_row)):
        mid = torch.zeros(total, max_rank, device=dev, dtype=dt)
        mid = sgemm_lora_a_fwd(x, a_stack, meta, mid)
        outs[tag] = sgemm_lora_b_fwd(mid, b_stack, meta, base_output=base.clone())
    torch.testing.assert_close(outs["group"], outs["row"], rtol=2e-2, atol=2e-2)
    assert torch.equal(outs["group"], outs["row"])


@pytest.mark.parametrize(
    "in_dim,out_dim,r_max,ranks",
    [
        (100, 1000, 16, [16, 5, 0]),     # unaligned rows, out not a multiple of 256, odd rank
        (16, 32, 8, [4, 8, 1]),          # tiny toy shapes
        (64, 128, 16, [8, 16, 3]),
        (4104, 520, 24, [24, 17, 9]),    # r_max not a power of two, in just past 4096
        (14336, 384, 64, [64, 48, 33]),  # long reduction -> split-K path
    ],
)
def test_odd_shapes_and_stale_tails(dev, in_dim, out_dim, r_max, ranks):
    """Stale data past each slot's rank (as a reused slot holds) must never be read."""
    g = torch.Generator().manual_seed(in_dim + out_dim)
    n_slots = len(ranks)
    lens = [3, 1, 0, 7, 2, 19]
    slots = [0, 1, 2, 1, 0, 2]
    x = torch.randn(sum(lens), in_dim, generator=g).bfloat16()
    a = (torch.randn(n_slots, r_max, in_dim, generator=g) * in_dim ** -0.5).bfloat16()
    b = (torch.randn(n_slots, out_dim, r_max, generator=g) * 0.05).bfloat16()
    base = torch.randn(sum(lens), out_dim, generator=g).bfloat16()
    scal = [1.5, 0.75, 2.0]
    meta_cpu = make_meta(lens, slots, ranks, scal, "cpu", torch.bfloat16)
    want = apply_f64(x, [a], [b], meta_cpu, base)
    kmid, kout = apply_kernel_numerics(x, [a], [b], meta_cpu, base)
    mid, out = run_hip(x.to(dev), [a.to(dev)], [b.to(dev)], make_meta(lens, slots, ranks, scal, dev, torch.bfloat16),
                       base.to(dev))
    assert_tol_f64(out, want)
    assert_ulp_close(out, kout, what="out")
    live = torch.zeros(sum(lens), dtype=torch.bool)
    st = 0
    for n, s in zip(lens, slots):
        live[st:st + n] = True
        st += n
    assert_ulp_close(mid[live], kmid[live], what="mid")


def test_rank0_empty_and_out_of_range_slots_leave_output_untouched(dev):
    dt = torch.bfloat16
    lens = [2, 0, 3, 1, 4]
    slots = [1, 0, 7, -1, 1]  # slot 1 has rank 0; 7 and -1 are outside the 3-slot pool
    ranks = [8, 0, 8]
    x = torch.randn(sum(lens), 64).to(dev, dt)
    a = torch.randn(3, 8, 64).to(dev, dt)
    b = torch.randn(3, 256, 8).to(dev, dt)
    base = torch.randn(sum(lens), 256).to(dev, dt)
    meta = make_meta(lens, slots, ranks, [1.0, 1.0, 1.0], dev, dt)
    mid, out = run_hip(x, [a], [b], meta, base)
    assert torch.equal(out, base.cpu())
    assert torch.count_nonzero(mid) == 0  # every row in a segment is written, and all are zero


def test_strided_output_view(dev):
    """Output is a column slice of a wider row (the fused-QKV case, row stride 6144)."""
    dt = torch.bfloat16
    wl = synthetic.decode_q(device=dev, tokens=24, in_dim=1024, out=1024, n_slots=8, n_adapters=6, rank=16, seed=5)
    wide = torch.randn(24, 6144, generator=torch.Generator().manual_seed(9)).to(dev, dt)
    view = wide[:, 4096:5120]
    assert not view.is_contiguous()
    before = wide.clone()
    mid = torch.empty(24, 16, device=dev, dtype=dt)
    sgemm_lora_a_fwd(wl.x, wl.a_stacks[0], wl.meta, mid)
    sgemm_lora_b_fwd(mid, wl.b_stacks[0], wl.meta, base_output=view)
    torch.cuda.synchronize()
    cm = cpu_meta(wl.meta)
    want = apply_f64(wl.x.cpu(), [wl.a_stacks[0].cpu()], [wl.b_stacks[0].cpu()], cm, before[:, 4096:5120].cpu())
    assert_tol_f64(wide[:, 4096:5120].cpu(), want)
    assert torch.equal(wide[:, :4096], before[:, :4096])
    assert torch.equal(wide[:, 5120:], before[:, 5120:])


def test_split_k_is_deterministic(dev):
    """A long reduction takes the split-K path; splits are summed in a fixed order."""
    wl = synthetic.prefill_mlp(device=dev, part="down", n_seg=3, min_len=5, max_len=40, hidden=512, inter=14336,
                               seed=4)
    first = run_hip(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, wl.base)
    for _ in range(3):
        again = run_hip(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, wl.base)
        assert torch.equal(first[0], again[0]) and torch.equal(first[1], again[1])
    check_workload(wl)


@pytest.mark.parametrize("n_short", [61, 150])
def test_mixed_long_and_one_row_segments(dev, n_short):
    """A mixed batch (long prefill segments among many one-row and empty ones,
    64 segments or more, so the dense tile map scans one full chunk of the
    segment table or several) through the fused three-slice path: every tile of every
    segment is computed once, rows of rank-0 and out-of-pool segments stay
    untouched."""
    g = torch.Generator().manual_seed(n_short)
    lens = [1] * n_short
    for pos, n in ((5, 70), (n_short // 2, 130), (n_short - 1, 200)):
        lens.insert(pos, n)
    lens[3] = 0
    lens[n_short // 3] = 0
    n_slots = 12
    slots = torch.randint(0, n_slots, (len(lens),), generator=g).tolist()
    slots[7], slots[n_short // 2 + 4] = -1, n_slots + 3
    ranks = [16] * n_slots
    ranks[2] = 0
    ranks[5] = 9
    in_dim, outs, r_max = 1024, [512, 128, 128], 16
    x = torch.randn(sum(lens), in_dim, generator=g).bfloat16()
    As = [(torch.randn(n_slots, r_max, in_dim, generator=g) * in_dim ** -0.5).bfloat16() for _ in outs]
    Bs = [(torch.randn(n_slots, o, r_max, generator=g) * 0.05).bfloat16() for o in outs]
    base = torch.randn(sum(lens), sum(outs), generator=g).bfloat16()
    cols = [0, outs[0], outs[0] + outs[1]]
    scal = [1.0 + 0.25 * i for i in range(n_slots)]
    meta_cpu = make_meta(lens, slots, ranks, scal, "cpu", torch.bfloat16)
    assert meta_cpu.bs >= 64 and meta_cpu.max_len > 16  # one full chunk of the table, or several
    want = apply_f64(x, As, Bs, meta_cpu, base, cols)
    kmid, kout = apply_kernel_numerics(x, As, Bs, meta_cpu, base, cols)
    mid, out = run_hip(x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs],
                       make_meta(lens, slots, ranks, scal, dev, torch.bfloat16), base.to(dev), cols)
    assert_tol_f64(out, want)
    assert_ulp_close(out, kout, what="out")
    assert_ulp_close(mid, kmid, what="mid")
    st = 0
    for n, s in zip(lens, slots):
        if not (0 <= s < n_slots) or ranks[s] == 0:
            assert torch.equal(out[st:st + n], base[st:st + n])
        st += n


@pytest.mark.parametrize("n_slices,r_max,ranks", [
    (1, 16, [16, 9, 0, 16]),     # one A block per stage (padded to two)
    (2, 16, [16, 5, 0, 12]),     # two blocks
    (3, 16, [16, 16, 0, 7]),     # three blocks, compiled as four
    (2, 64, [64, 40, 0, 17]),    # eight blocks
    (3, 64, [64, 40, 0, 17]),    # twelve blocks: q|k, then v, one launch each
    (4, 48, [48, 33, 0, 7]),     # twelve blocks of three per slice: two launches of two slices
    (1, 18, [18, 5, 0, 11]),     # r_max not a multiple of 4: split sums stored a column at a time
])
def test_streamed_lds_shrink_block_counts(dev, n_slices, r_max, ranks):
    """Long segments with K a multiple of 64 take the shrink that streams x
    and A straight into LDS; every block count it compiles, with the K
    reduction split over workgroups, ranks below r_max, a rank-0 slot and
    tiles shorter than 64 rows."""
    g = torch.Generator().manual_seed(n_slices * 100 + r_max)
    in_dim, outs = 8192, [256] * n_slices
    lens = [70, 3, 130, 64, 20]
    slots = [0, 2, 1, 3, 0]
    n_slots = len(ranks)
    x = torch.randn(sum(lens), in_dim, generator=g).bfloat16()
    As = [(torch.randn(n_slots, r_max, in_dim, generator=g) * in_dim ** -0.5).bfloat16() for _ in outs]
    Bs = [(torch.randn(n_slots, o, r_max, generator=g) * 0.05).bfloat16() for o in outs]
    base = torch.randn(sum(lens), sum(outs), generator=g).bfloat16()
    cols = [256 * s for s in range(n_slices)]
    scal = [0.5, 1.0, 1.5, 2.0]
    meta_cpu = make_meta(lens, slots, ranks, scal, "cpu", torch.bfloat16)
    want = apply_f64(x, As, Bs, meta_cpu, base, cols)
    kmid, kout = apply_kernel_numerics(x, As, Bs, meta_cpu, base, cols)
    mid, out = run_hip(x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs],
                       make_meta(lens, slots, ranks, scal, dev, torch.bfloat16), base.to(dev), cols)
    assert_tol_f64(out, want)
    assert_ulp_close(out, kout, what="out")
    assert_ulp_close(mid, kmid, what="mid")


class _OffsetWorkspace:
    """A workspace whose pointer is `offset` bytes past a fresh allocation."""

    def __init__(self, offset):
        self.offset, self.buf = offset, None

    def get(self, need, dev):
        self.buf = torch.empty(need + 256, dtype=torch.uint8, device=dev)
        return self.buf.data_ptr() + self.offset, need


def test_streamed_shrink_split_sums_in_an_unaligned_workspace(dev):
    """The streamed shrink stores its split sums 16 bytes at a time when the
    workspace allows it, and a column at a time when the caller's workspace
    is only 4-byte aligned: the results are the same bit for bit."""
    wl = synthetic.prefill_mlp(device=dev, part="gate_up", n_seg=4, min_len=64, max_len=200, hidden=4096,
                               inter=1024, seed=11)
    r_max = wl.a_stacks[0].shape[1]
    outs = []
    for ws in (None, _OffsetWorkspace(4), _OffsetWorkspace(8)):
        mid = torch.full((wl.x.shape[0], len(wl.a_stacks) * r_max), float("nan"), dtype=wl.x.dtype, device=dev)
        if ws is None:
            sgemm_lora_a_multi_fwd(wl.x, wl.a_stacks, wl.meta, mid)
        else:
            shrink(wl.x, wl.a_stacks, wl.meta, mid, workspace=ws)
        torch.cuda.synchronize()
        outs.append(mid.cpu())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    kmid, _ = apply_kernel_numerics(wl.x.cpu(), [a.cpu() for a in wl.a_stacks], [b.cpu() for b in wl.b_stacks],
                                    cpu_meta(wl.meta), wl.base.cpu(), wl.col_offsets)
    assert_ulp_close(outs[0], kmid, what="mid")


@pytest.mark.parametrize("scal_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_streamed_paths_skip_out_of_pool_and_rank0_slots(dev, scal_dtype):
    """Long segments take the streamed shrink and expand; the streamed
    expand requests a tile's B and output rows before the slot's rank has
    arrived (B through the slot clamped to the pool).  Slots outside the
    pool on both sides and a rank-0 slot leave their rows as they were;
    slots of both parities read a 16-bit scaling from either half of its
    32-bit word.  Two calls and the one-call path agree bit for bit."""
    g = torch.Generator().manual_seed(77)
    in_dim, out_dim, r_max = 4096, 512, 32
    lens = [130, 70, 96, 64, 150, 90]
    slots = [1, -1, 0, 5, 3, 2]  # pool of 4: -1 and 5 lie outside it; slot 0 has rank 0
    ranks = [0, 32, 16, 8]
    scal = [0.75, 1.5, 2.0, 0.5]
    rows = sum(lens)
    assert rows >= 64 * len(lens)  # the streamed (long-segment) kernels
    x = torch.randn(rows, in_dim, generator=g).bfloat16()
    a = (torch.randn(len(ranks), r_max, in_dim, generator=g) * in_dim ** -0.5).bfloat16()
    b = (torch.randn(len(ranks), out_dim, r_max, generator=g) * 0.05).bfloat16()
    base = torch.randn(rows, out_dim, generator=g).bfloat16()
    meta_cpu = make_meta(lens, slots, ranks, scal, "cpu", scal_dtype)
    want = apply_f64(x, [a], [b], meta_cpu, base)
    kmid, kout = apply_kernel_numerics(x, [a], [b], meta_cpu, base)
    meta = make_meta(lens, slots, ranks, scal, dev, scal_dtype)
    mid, out = run_hip(x.to(dev), [a.to(dev)], [b.to(dev)], meta, base.to(dev))
    assert_tol_f64(out, want)
    assert_ulp_close(out, kout, what="out")
    one = base.to(dev)
    apply_segments(x.to(dev), [a.to(dev)], [b.to(dev)], meta, one, [0])
    torch.cuda.synchronize()
    assert torch.equal(one.cpu(), out)
    st = 0
    for n, slot in zip(lens, slots):
        if not 0 <= slot < len(ranks) or ranks[slot] == 0:
            assert torch.equal(out[st:st + n], base[st:st + n]), (slot, st)
            assert torch.count_nonzero(mid[st:st + n]) == 0, (slot, st)
        else:
            assert not torch.equal(out[st:st + n], base[st:st + n]), (slot, st)
        st += n


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_streamed_expand_long_segments(dev, dtype):
    """Segments of 64 rows or more on average take the expand that stages the
    output tile in LDS (64-row tiles): slices of 1000 and 264 columns (partial
    column tiles) at an offset inside a wider output row, a rank-0 slot,
    ranks below r_max and segment lengths that are not multiples of 64."""
    g = torch.Generator().manual_seed(77)
    in_dim, r_max = 512, 32
    outs = [1000, 264]
    lens = [150, 65, 200, 63, 130]
    slots = [1, 0, 3, 2, 1]
    ranks = [32, 0, 20, 9]
    n_slots = len(ranks)
    assert sum(lens) >= 64 * len(lens)
    x = torch.randn(sum(lens), in_dim, generator=g).to(dtype)
    As = [(torch.randn(n_slots, r_max, in_dim, generator=g) * in_dim ** -0.5).to(dtype) for _ in outs]
    Bs = [(torch.randn(n_slots, o, r_max, generator=g) * 0.05).to(dtype) for o in outs]
    wide = torch.randn(sum(lens), 1400, generator=g).to(dtype)
    cols = [8, 8 + outs[0]]
    scal = [1.5, 1.0, 0.5, 2.0]
    meta_cpu = make_meta(lens, slots, ranks, scal, "cpu", dtype)
    want = apply_f64(x, As, Bs, meta_cpu, wide, cols)
    kmid, kout = apply_kernel_numerics(x, As, Bs, meta_cpu, wide, cols)
    mid, out = run_hip(x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs],
                       make_meta(lens, slots, ranks, scal, dev, dtype), wide.to(dev), cols)
    assert_tol_f64(out, want)
    assert_ulp_close(out, kout, what="out")
    assert_ulp_close(mid, kmid, what="mid")
    assert torch.equal(out[:, :8], wide[:, :8]) and torch.equal(out[:, 8 + sum(outs):], wide[:, 8 + sum(outs):])
    st = 0
    for n, slot in zip(lens, slots):
        if ranks[slot] == 0:  # rank-0 slot: its segments' rows are untouched
            assert torch.equal(out[st:st + n], wide[st:st + n])
        st += n


@pytest.mark.parametrize("part", ["qkv", "gate_up", "o", "down"])
def test_c5_mixed_batch_full_shape(dev, part):
    """The 32-layer step's batch at its real shape: 2 x 512 prefill rows and
    64 one-row decode segments (1088 rows, 66 segments) through the fused
    q|k|v (4096 -> 4096/1024/1024), the fused gate|up (4096 -> 2 x 14336:
    streamed long tiles interleaved with the short items), the o projection
    (4096 -> 4096) or the down projection (14336 -> 4096; o and down add the
    split sums in the expand), rank 16 in a 128-slot pool with adapters
    drawn Zipf(1.1) over 512."""
    g = torch.Generator().manual_seed(4)
    lens = [512, 512] + [1] * 64
    zipf = torch.tensor([(i + 1) ** -1.1 for i in range(512)])
    picks = torch.multinomial(zipf, len(lens), replacement=True, generator=g).tolist()
    first = {}
    slots = [first.setdefault(p, len(first)) for p in picks]
    n_slots, r = 128, 16
    ranks = [r] * len(first) + [0] * (n_slots - len(first))
    in_dim, outs = {"qkv": (4096, [4096, 1024, 1024]), "gate_up": (4096, [14336, 14336]), "o": (4096, [4096]),
                    "down": (14336, [4096])}[part]
    used = sorted(set(slots))
    x = torch.randn(sum(lens), in_dim, generator=g).bfloat16()
    As, Bs = [], []
    for o in outs:
        a = torch.zeros(n_slots, r, in_dim, dtype=torch.bfloat16)
        b = torch.zeros(n_slots, o, r, dtype=torch.bfloat16)
        a[used] = (torch.randn(len(used), r, in_dim, generator=g) * in_dim ** -0.5).bfloat16()
        b[used] = (torch.randn(len(used), o, r, generator=g) * 0.02).bfloat16()
        As.append(a)
        Bs.append(b)
    base = torch.randn(sum(lens), sum(outs), generator=g).bfloat16()
    cols = [sum(outs[:i]) for i in range(len(outs))]
    meta_cpu = make_meta(lens, slots, ranks, [2.0] * n_slots, "cpu", torch.bfloat16)
    want = apply_f64(x, As, Bs, meta_cpu, base, cols)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    meta = make_meta(lens, slots, ranks, [2.0] * n_slots, dev, torch.bfloat16)
    mid, out = run_hip(xd, Ad, Bd, meta, base.to(dev), cols)
    assert_tol_f64(out, want, f"c5 {part}")
    # The backend's one-call path (the expand adds the split sums itself for
    # o and down) equals the two-call path element for element.
    one = base.to(dev)
    apply_segments(xd, Ad, Bd, meta, one, cols, workspace=Workspace())
    torch.cuda.synchronize()
    assert torch.equal(one.cpu(), out), f"c5 {part}: one call differs from shrink then expand"
