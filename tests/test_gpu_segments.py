"""One-call segment shrink + expand (mlora_apply_segments) on the GPU.

The call must equal the two-call path (mlora_shrink into a caller `mid`,
then mlora_expand) element for element, whether the expand reads `mid` or
adds up the shrink's split sums itself (split K, 16-bit data, r_max <= 64,
segments not all long), and must match the oracle like every other path.
"""

import pytest
import torch

from multi_lora_amd import HipLoRABackend
from multi_lora_amd.kernels.lora_ops import Workspace, apply_segments
from multi_lora_amd.synthetic import make_meta
from oracle.lora_ref import apply_f64
from tests.gpu_helpers import assert_tol_f64
from tests.test_gpu_lora import run_hip

pytestmark = pytest.mark.gpu


def case(dev, lens, slots, ranks, in_dim, outs, r_max, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    n_slots = len(ranks)
    x = torch.randn(sum(lens), in_dim, generator=g).to(dtype)
    As = [(torch.randn(n_slots, r_max, in_dim, generator=g) * in_dim ** -0.5).to(dtype) for _ in outs]
    Bs = [(torch.randn(n_slots, o, r_max, generator=g) * 0.05).to(dtype) for o in outs]
    base = torch.randn(sum(lens), sum(outs), generator=g).to(dtype)
    cols = [sum(outs[:i]) for i in range(len(outs))]
    scal = [0.5 + 0.25 * i for i in range(n_slots)]
    return x, As, Bs, base, cols, make_meta(lens, slots, ranks, scal, "cpu", dtype), scal


@pytest.mark.parametrize("name,lens,slots,ranks,in_dim,outs,r_max,dtype", [
    # mixed batch, split K: the expand adds the split sums itself
    ("mixed", [70] + [1] * 40 + [130], [0] + [i % 5 for i in range(40)] + [3], [16, 16, 0, 9, 16], 4096,
     [512, 128, 128], 16, torch.bfloat16),
    ("mixed_r64", [90, 1, 1, 3, 40, 1], [0, 1, 2, 0, 3, 1], [64, 33, 0, 48], 8192, [256, 256], 64, torch.float16),
    ("decode_split", [1] * 24 + [5], [i % 6 for i in range(25)], [16, 8, 16, 0, 16, 12], 8192, [384], 16,
     torch.bfloat16),
    # long segments (streamed expand reads mid), fp32 (no split sums), K not split
    ("long", [150, 200, 130], [0, 1, 0], [16, 32], 4096, [1024, 256], 32, torch.bfloat16),
    ("fp32", [20, 1, 33], [0, 1, 0], [8, 16], 1024, [256], 16, torch.float32),
    ("short_k", [30, 2, 17], [1, 0, 1], [16, 16], 64, [128], 16, torch.bfloat16),
    # r_max % 8 == 4 with split K: the expand's y tile is a chunk wider than
    # r_max, and the chunk's tail must not reach the MFMA unmasked
    ("rmax4_split", [1] * 24 + [3], [i % 5 for i in range(25)], [4, 4, 0, 3, 4], 4096, [512], 4, torch.bfloat16),
    ("rmax4_split_f16", [2] * 20, [i % 3 for i in range(20)], [4, 2, 4], 4096, [264], 4, torch.float16),
    ("rmax12_split", [1] * 30, [i % 6 for i in range(30)], [12, 12, 7, 0, 12, 5], 4096, [640], 12, torch.float16),
    ("rmax12_mixed_bf16", [40] + [1] * 20 + [33], [0] + [i % 4 for i in range(20)] + [2], [12, 9, 12, 4], 4096,
     [512, 256], 12, torch.bfloat16),
    # q|k|v at r_max 64 (twelve A blocks): the shrink runs once per group of
    # slices (q|k, then v), each writing its columns of mid / the split sums
    ("qkv_r64_mixed", [90, 1, 1, 3, 40, 1], [0, 1, 2, 0, 3, 1], [64, 33, 0, 48], 4096, [512, 128, 128], 64,
     torch.bfloat16),
    ("qkv_r64_decode", [1] * 24 + [5], [i % 6 for i in range(25)], [64, 17, 64, 0, 40, 64], 4096, [512, 128, 128],
     64, torch.bfloat16),
    ("qkv_r64_long", [150, 200, 130], [0, 1, 0], [64, 40], 4096, [512, 128, 128], 64, torch.float16),
    # long reductions over long segments: the streamed shrink's 128-row tiles
    ("long_k8192", [300, 520, 280], [0, 1, 2], [64, 16, 40], 8192, [1024, 256], 64, torch.bfloat16),
    ("long_k14336_f16", [260, 1, 400], [1, 2, 0], [32, 64, 0], 14336, [512], 64, torch.float16),
])
def test_one_call_equals_two_calls(dev, name, lens, slots, ranks, in_dim, outs, r_max, dtype):
    x, As, Bs, base, cols, meta_cpu, scal = case(dev, lens, slots, ranks, in_dim, outs, r_max, dtype, len(name))
    meta = make_meta(lens, slots, ranks, scal, dev, dtype)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    _, two = run_hip(xd, Ad, Bd, meta, base.to(dev), cols)
    one = base.to(dev).clone()
    apply_segments(xd, Ad, Bd, meta, one, cols, workspace=Workspace())
    torch.cuda.synchronize()
    assert torch.equal(one.cpu(), two), f"{name}: one-call result differs from shrink + expand"
    assert not torch.isnan(one).any().item(), name
    assert_tol_f64(one.cpu(), apply_f64(x, As, Bs, meta_cpu, base, cols), name)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_long_k_rows_not_16_byte_aligned(dev, dtype):
    """A batch that plans the streamed shrink's 128-row tiles, with x rows
    4 elements apart from 16-byte alignment: the register-staged kernels run
    it on 64-row tiles instead, with the same results as aligned rows."""
    lens, slots, ranks, in_dim, outs, r_max = [300, 1, 420], [0, 1, 2], [64, 16, 48], 8192, [768], 64
    x, As, Bs, base, cols, meta_cpu, scal = case(dev, lens, slots, ranks, in_dim, outs, r_max, dtype, 77)
    meta = make_meta(lens, slots, ranks, scal, dev, dtype)
    Ad, Bd = [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    padded = torch.zeros(x.shape[0], in_dim + 4, dtype=dtype, device=dev)
    padded[:, :in_dim] = x.to(dev)
    xs = padded[:, :in_dim]
    assert xs.stride(0) % 8 != 0
    got = base.to(dev).clone()
    apply_segments(xs, Ad, Bd, meta, got, cols, workspace=Workspace())
    aligned = base.to(dev).clone()
    apply_segments(x.to(dev), Ad, Bd, meta, aligned, cols, workspace=Workspace())
    torch.cuda.synchronize()
    assert_tol_f64(got.cpu(), apply_f64(x, As, Bs, meta_cpu, base, cols), f"unaligned {dtype}")
    assert_tol_f64(aligned.cpu(), apply_f64(x, As, Bs, meta_cpu, base, cols), f"aligned {dtype}")


@pytest.mark.parametrize("name,lens,slots,ranks,in_dim,outs,r_max,dtype", [
    # split K with an output too wide for the expand to add the split sums:
    # the split reduce fills the call's own mid over every row and column
    ("wide_mixed", [70] + [1] * 30 + [130], [0] + [i % 5 for i in range(30)] + [3], [32, 16, 0, 9, 32], 4096,
     [4096, 512], 32, torch.bfloat16),
    # long segments (the streamed expand reads mid), a rank-0 slot, an empty
    # segment, ranks below r_max
    ("long_ranks", [150, 200, 0, 130, 90], [0, 1, 2, 3, 1], [16, 0, 48, 64], 8192, [1024, 256], 64,
     torch.float16),
])
@pytest.mark.parametrize("fill", [0xFF, 0x7F])
def test_apply_ignores_what_the_workspace_held(dev, name, lens, slots, ranks, in_dim, outs, r_max, dtype, fill):
    """The apply path's split reduce writes its private mid over every row and
    column, stale split sums included (rank-0 rows, columns past a rank,
    rows no segment covers).  With the workspace's bytes set beforehand to
    0xFF (fp32 NaN) or 0x7F (3.4e38, whose sums overflow), the output equals
    the zeroed workspace's and the two-call path's bit for bit, and the rows
    past the table keep their base values."""
    extra = 7
    x, As, Bs, base, cols, meta_cpu, scal = case(dev, lens + [extra], slots + [0], ranks, in_dim, outs, r_max, dtype,
                                                 len(name))
    meta = make_meta(lens, slots, ranks, scal, dev, dtype)
    meta_cpu = make_meta(lens, slots, ranks, scal, "cpu", dtype)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    zeroed = base.to(dev).clone()
    apply_segments(xd, Ad, Bd, meta, zeroed, cols, workspace=Workspace())
    stale_ws = Workspace()
    stale_ws.buf = torch.full((64 << 20,), fill, dtype=torch.uint8, device=dev)
    stale = base.to(dev).clone()
    apply_segments(xd, Ad, Bd, meta, stale, cols, workspace=stale_ws)
    torch.cuda.synchronize()
    assert torch.equal(stale.cpu(), zeroed.cpu()), f"{name}: the workspace's old bytes reached the output"
    _, two = run_hip(xd, Ad, Bd, meta, base.to(dev), cols)
    assert torch.equal(zeroed.cpu(), two), f"{name}: one-call result differs from shrink + expand"
    assert torch.equal(stale.cpu()[sum(lens):], base[sum(lens):]), f"{name}: rows past the table changed"
    assert_tol_f64(stale.cpu(), apply_f64(x, As, Bs, meta_cpu, base, cols), name)


@pytest.mark.parametrize("r_max", [4, 12])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_backend_decode_at_rank_widths_the_grouped_path_refuses(dev, r_max, dtype):
    """Decode batches whose r_max is not a multiple of 8 go to the one-call
    segment path; at in_dim 4096 its expand adds the split sums itself.
    The result has no NaN, equals shrink + expand and matches float64."""
    lens = [1] * 40
    slots = [(7 * i) % 6 for i in range(40)]
    ranks = [r_max, r_max - 1, 0, r_max, 2, r_max]
    x, As, Bs, base, cols, meta_cpu, scal = case(dev, lens, slots, ranks, 4096, [1024], r_max, dtype, r_max)
    meta = make_meta(lens, slots, ranks, scal, dev, dtype)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    be = HipLoRABackend()
    be.set_kernel_input_metadata(meta)
    got = be.apply_lora(xd, Ad[0], Bd[0], base.to(dev).clone())
    _, two = run_hip(xd, Ad, Bd, meta, base.to(dev), cols)
    torch.cuda.synchronize()
    assert not torch.isnan(got).any().item()
    assert torch.equal(got.cpu(), two)
    assert_tol_f64(got.cpu(), apply_f64(x, As, Bs, meta_cpu, base, cols), f"r_max {r_max}")


def test_backend_mixed_batch_uses_one_call_and_replays_in_a_graph(dev):
    """The backend's apply_lora_multi on a mixed batch, eager and under HIP
    graph replay (several replays with a metadata rewrite in between), equals
    the two-call path each time."""
    lens = [64] + [1] * 30
    slots = [0] + [i % 4 for i in range(30)]
    ranks = [16, 16, 16, 16]
    x, As, Bs, base, cols, _, scal = case(dev, lens, slots, ranks, 4096, [1024, 256], 16, torch.bfloat16, 5)
    meta = make_meta(lens, slots, ranks, scal, dev, torch.bfloat16)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    be = HipLoRABackend()
    be.set_kernel_input_metadata(meta)
    out = base.to(dev).clone()
    be.apply_lora_multi(xd, Ad, Bd, out, cols)
    _, want = run_hip(xd, Ad, Bd, meta, base.to(dev), cols)
    assert torch.equal(out.cpu(), want)
    out.copy_(base.to(dev))
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        be.apply_lora_multi(xd, Ad, Bd, out, cols)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        be.apply_lora_multi(xd, Ad, Bd, out, cols)
    for rep in range(3):
        out.copy_(base.to(dev))
        if rep == 2:  # rewrite the slots in place: the replay must follow
            meta.weight_indices.copy_(torch.tensor([1] + [(i + 1) % 4 for i in range(30)], dtype=torch.int32))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _, want = run_hip(xd, Ad, Bd, meta, base.to(dev), cols)
        assert torch.equal(out.cpu(), want), f"replay {rep}"


def zipf_slots(g, n, n_adapters, n_slots):
    """Slots of n requests drawn Zipf(1.1) over n_adapters adapters, the
    adapters placed in pool slots in order of first appearance."""
    zipf = torch.tensor([(i + 1) ** -1.1 for i in range(n_adapters)])
    picks = torch.multinomial(zipf, n, replacement=True, generator=g).tolist()
    first = {}
    return [first.setdefault(p, len(first)) % n_slots for p in picks]


MIXED_CASES = [
    # name, lens, slots (None: Zipf), ranks, in_dim, outs, r_max, dtype
    # wide outputs: the expand reads mid; two long segments and 64 one-row ones
    ("wide_mid", [512, 512] + [1] * 64, None, [16] * 48 + [0] * 16, 1024, [4096, 1024, 1024], 16, torch.bfloat16),
    # narrow output with split K: the expand adds the split sums
    ("narrow_split", [300, 90] + [1] * 40, None, [16] * 40, 4096, [1024], 16, torch.bfloat16),
    # r_max 64, ranks below it (stale tails), fp16, short segments of 2..16 rows
    ("r64_f16", [200, 40, 3, 16, 7, 1, 2, 17, 9, 1, 5, 0, 12],
     [0, 1, 2, 3, 2, 0, 1, 4, 3, 2, 5, 1, 0], [64, 40, 16, 33, 64, 8], 2048, [768, 512], 64, torch.float16),
    # rank-0, out-of-pool and empty short segments next to live ones
    ("odd_slots", [100, 1, 1, 4, 1, 0, 3, 1, 33], [0, 9, -1, 1, 2, 1, 1, 3, 2], [16, 16, 0, 16], 1024, [512], 16,
     torch.bfloat16),
    # wide enough for 64-row long tiles streamed through LDS (17 row tiles x
    # 112 column tiles, at least four workgroups a CU on a 256-CU GPU)
    ("gate_up_streamed", [512, 512] + [1] * 64, None, [16] * 48 + [0] * 16, 1024, [14336, 14336], 16,
     torch.bfloat16),
    # streamed, fp16: ragged long segments (not multiples of 64 rows; ranks
    # 32, 0, 24, 8), short ones of 1..16 rows, ranks below r_max
    ("ragged_streamed_f16", [700, 333, 5, 70, 1, 16, 17, 2, 1, 9] + [1] * 30,
     [0, 2, 5, 1, 3, 6, 4, 7, 9, 10] + [(7 * i) % 64 for i in range(30)],
     [32, 24, 0, 32, 8, 16, 32, 24] * 8, 1024, [12288, 12288], 32, torch.float16),
    # streamed at r_max 64 (two MFMA K-steps)
    ("r64_streamed", [640, 384] + [1, 2, 3, 16] * 10, None, [64, 40, 16, 0] * 16, 1024, [14336, 14336], 64,
     torch.bfloat16),
]


@pytest.mark.parametrize("name,lens,slots,ranks,in_dim,outs,r_max,dtype", MIXED_CASES)
def test_mixed_batch_expand_equals_tiled(dev, name, lens, slots, ranks, in_dim, outs, r_max, dtype):
    """With the host summary, a batch mixing long and short segments takes
    the one-launch mixed expand (slot-grouped items for the short segments);
    without it, every segment is tiled.  Results are equal bit for bit, also
    when the summary is wrong (too small: units loop; too large: units exit),
    and match the oracle.  A summary of 5/8 of the long rows in one segment
    keeps the streamed cases streamed, with too few units: the extra tiles
    go as 32-row halves."""
    g = torch.Generator().manual_seed(len(name))
    if slots is None:
        slots = [0] * 2 + zipf_slots(g, len(lens) - 2, 512, len(ranks))
    x, As, Bs, base, cols, meta_cpu, scal = case(dev, lens, slots, ranks, in_dim, outs, r_max, dtype, len(name))
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]

    def run(meta):
        out = base.to(dev).clone()
        apply_segments(xd, Ad, Bd, meta, out, cols, workspace=Workspace())
        torch.cuda.synchronize()
        return out.cpu()

    tiled = run(make_meta(lens, slots, ranks, scal, dev, dtype, host_copies=False))
    hinted = make_meta(lens, slots, ranks, scal, dev, dtype)
    long_segs, long_rows, short_slots = hinted.table_summary(len(ranks))
    assert long_segs > 0 and short_slots > 0, "the case must mix long and short segments"
    assert torch.equal(run(hinted), tiled), f"{name}: mixed expand differs from the tiled one"
    for wrong in ((1, 1, 1), (long_segs, long_rows, max(1, short_slots // 3)),
                  (long_segs + 5, long_rows + 900, short_slots + 7), (1, max(1, long_rows * 5 // 8), short_slots)):
        bad = make_meta(lens, slots, ranks, scal, dev, dtype)
        bad.table_summary = lambda n, w=wrong: w
        assert torch.equal(run(bad), tiled), f"{name}: summary {wrong} changed the result"
    assert_tol_f64(tiled, apply_f64(x, As, Bs, meta_cpu, base, cols), name)


@pytest.mark.parametrize("n_slots", [2048, 2049])
def test_mixed_batch_expand_at_the_pool_size_limit(dev, n_slots):
    """The mixed expand keeps the distinct short slots as a bitmap of 2048
    slots in LDS: at 2048 slots it runs with short segments on slots at the
    bitmap's word boundaries (31/32/33, 63/64, 1023/1024, 2047) and equals
    the tiled result bit for bit; at 2049 slots the call takes the tiled
    path.  Both match the oracle."""
    short_slots = [0, 31, 32, 33, 63, 64, 1023, 1024, 2016, 2047, 32, 1024, 5, 2046]
    lens = [100, 70] + [1, 3, 1, 16, 1, 2, 1, 1, 5, 1, 1, 9, 1, 1]
    slots = [2047, 5] + short_slots
    ranks = [16] * n_slots
    ranks[33] = 0
    ranks[1023] = 8
    x, As, Bs, base, cols, _, _ = case(dev, lens, slots, ranks, 256, [512], 16, torch.bfloat16, 21)
    # Scalings in the usual range (the helper's grow with the slot number).
    scal = [0.5 + 0.25 * (i % 8) for i in range(n_slots)]
    meta_cpu = make_meta(lens, slots, ranks, scal, "cpu", torch.bfloat16)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]

    def run(meta):
        out = base.to(dev).clone()
        apply_segments(xd, Ad, Bd, meta, out, cols, workspace=Workspace())
        torch.cuda.synchronize()
        return out.cpu()

    hinted = make_meta(lens, slots, ranks, scal, dev, torch.bfloat16)
    long_segs, _, n_short = hinted.table_summary(n_slots)
    assert long_segs == 2 and n_short == len(set(short_slots))
    got = run(hinted)
    assert torch.equal(got, run(make_meta(lens, slots, ranks, scal, dev, torch.bfloat16, host_copies=False)))
    assert_tol_f64(got, apply_f64(x, As, Bs, meta_cpu, base, cols), f"{n_slots} slots")


def test_interleaved_mixed_expand_in_a_replayed_graph_follows_table_rewrites(dev):
    """A wide mixed expand (2 x 14336 columns) whose short items exceed a round
    of workgroup slots interleaves long and short units and launches half as
    many short units as short slots.  Captured with 10 short slots, it is
    replayed after rewrites to 40 and back to 10, and each replay equals
    the tiled result."""
    g = torch.Generator().manual_seed(78)
    lens = [512, 300] + [1] * 40
    ranks = [16] * 64
    slots0 = [0, 1] + [2 + (i % 10) for i in range(40)]            # 10 distinct short slots
    slots1 = [0, 1] + [20 + i for i in range(40)]                  # 40 after the rewrite
    x, As, Bs, base, cols, _, scal = case(dev, lens, slots0, ranks, 512, [14336, 14336], 16, torch.bfloat16, 4)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    meta = make_meta(lens, slots0, ranks, scal, dev, torch.bfloat16)
    assert meta.table_summary(64)[2] == 10
    out = base.to(dev).clone()
    ws = Workspace()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        apply_segments(xd, Ad, Bd, meta, out, cols, workspace=ws)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        apply_segments(xd, Ad, Bd, meta, out, cols, workspace=ws)
    for rep, slots in enumerate((slots0, slots1, slots0)):
        meta.weight_indices.copy_(torch.tensor(slots, dtype=torch.int32))
        meta.set_host_copies(lens, slots)
        out.copy_(base.to(dev))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = base.to(dev).clone()
        apply_segments(xd, Ad, Bd, make_meta(lens, slots, ranks, scal, dev, torch.bfloat16, host_copies=False), want,
                       cols, workspace=Workspace())
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), want.cpu()), f"replay {rep}"


def test_split_reduce_in_a_replayed_graph_follows_table_rewrites(dev):
    """Split K with an output too wide for the expand to add the split sums:
    the call runs the shrink, the table-free split reduce and the expand.
    Captured once, replayed after in-place rewrites of the slots (one of
    them moves segments to rank-0 slots, whose rows' reduced values are
    never read), each replay equals a fresh eager call."""
    lens = [300, 200] + [1] * 30
    ranks = [16] * 32 + [0] * 32
    slots0 = [0, 1] + [2 + (i % 8) for i in range(30)]
    slots1 = [40, 1] + [20 + (i % 16) + (i % 2) * 20 for i in range(30)]
    x, As, Bs, base, cols, _, scal = case(dev, lens, slots0, ranks, 4096, [4096, 1024], 16, torch.bfloat16, 9)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    meta = make_meta(lens, slots0, ranks, scal, dev, torch.bfloat16)
    out = base.to(dev).clone()
    ws = Workspace()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        apply_segments(xd, Ad, Bd, meta, out, cols, workspace=ws)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        apply_segments(xd, Ad, Bd, meta, out, cols, workspace=ws)
    for rep, slots in enumerate((slots0, slots1, slots0)):
        meta.weight_indices.copy_(torch.tensor(slots, dtype=torch.int32))
        meta.set_host_copies(lens, slots)
        out.copy_(base.to(dev))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = base.to(dev).clone()
        apply_segments(xd, Ad, Bd, make_meta(lens, slots, ranks, scal, dev, torch.bfloat16, host_copies=False), want,
                       cols, workspace=Workspace())
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), want.cpu()), f"replay {rep}"
        assert_tol_f64(out.cpu(), apply_f64(x, As, Bs, make_meta(lens, slots, ranks, scal, "cpu", torch.bfloat16),
                                            base, cols), f"replay {rep}")


def test_mixed_batch_expand_in_a_replayed_graph_follows_table_rewrites(dev):
    """A captured mixed expand keeps the launch size of its capture; after an
    in-place rewrite that gives the short segments more distinct slots, the
    replay still equals the tiled result (the kernel recounts and loops)."""
    g = torch.Generator().manual_seed(77)
    lens = [256, 200] + [1] * 48
    ranks = [16] * 64
    slots0 = [0, 1] + [2 + (i % 4) for i in range(48)]          # 4 distinct short slots at capture
    slots1 = [0, 1] + zipf_slots(g, 48, 64, 64)                   # many more after the rewrite
    x, As, Bs, base, cols, _, scal = case(dev, lens, slots0, ranks, 2048, [4096, 1024], 16, torch.bfloat16, 3)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    meta = make_meta(lens, slots0, ranks, scal, dev, torch.bfloat16)
    assert meta.table_summary(64)[2] == 4
    out = base.to(dev).clone()
    ws = Workspace()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        apply_segments(xd, Ad, Bd, meta, out, cols, workspace=ws)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        apply_segments(xd, Ad, Bd, meta, out, cols, workspace=ws)
    for rep, slots in enumerate((slots0, slots1, slots1, slots0)):
        meta.weight_indices.copy_(torch.tensor(slots, dtype=torch.int32))
        meta.set_host_copies(lens, slots)
        out.copy_(base.to(dev))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = base.to(dev).clone()
        apply_segments(xd, Ad, Bd, make_meta(lens, slots, ranks, scal, dev, torch.bfloat16, host_copies=False), want,
                       cols, workspace=Workspace())
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), want.cpu()), f"replay {rep}"
