"""RMSNorm folded into the slot-grouped decode apply (mlora_rmsnorm_apply_grouped), GPU.

The fused call writes y = RMSNorm(x), the same bits as the RMSNorm kernel,
and applies the LoRA to y without reading y: its shrink multiplies
round(x * w) with A and scales each row's sums by that row's
rsqrt(mean(x^2) + eps).  So y is held bit for bit to rmsnorm_fwd, and the
output to the float64 closed form of RMSNorm followed by the LoRA (the
reference's tolerance) and to one unit of the fused rounding sequence
(oracle.rmsnorm_ref.rmsnorm_shrink_input fed to the kernels' rounding
model).  Rows are scaled over four decades so that a missing or misplaced
rstd cannot pass.
"""

import pytest
import torch

from multi_lora_amd import synthetic
from multi_lora_amd.synthetic import make_meta
from multi_lora_amd.kernels.lora_ops import LinkedWorkspace, apply_grouped, rmsnorm_apply_grouped
from multi_lora_amd.kernels.rmsnorm import rmsnorm_fwd
from oracle.lora_ref import apply_f64, apply_kernel_numerics
from oracle.rmsnorm_ref import rmsnorm_f64, rmsnorm_shrink_input
from tests.gpu_helpers import assert_tol_f64, assert_ulp_close
from tests.test_gpu_grouped import workload
from tests.test_gpu_lora import cpu_meta

pytestmark = pytest.mark.gpu


def scaled(x: torch.Tensor, seed: int) -> torch.Tensor:
    """x with row i scaled by 10**u, u uniform in [-2, 2]."""
    g = torch.Generator().manual_seed(seed)
    s = 10.0 ** (torch.rand(x.shape[0], 1, generator=g) * 4 - 2)
    return (x.cpu().float() * s).to(x.dtype).to(x.device)


def norm_weight(n: int, dtype, dev, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=g) * 0.1 + 1.0).to(dtype).to(dev)


def fused(wl, x, w, eps, lws=None, split=False, meta=None):
    y = torch.empty_like(x)
    out = wl.clone_base()
    lws = lws if lws is not None else LinkedWorkspace()
    meta = wl.meta if meta is None else meta
    args = (x, w, eps, y, wl.a_stacks, wl.b_stacks, meta, out, wl.col_offsets, lws)
    if split:
        assert rmsnorm_apply_grouped(*args, phases=1)
        assert rmsnorm_apply_grouped(*args, phases=2)
    else:
        assert rmsnorm_apply_grouped(*args)
    torch.cuda.synchronize()
    _, pe = lws.counters()
    assert pe == 0, f"{pe} plan errors"
    return y.cpu(), out.cpu()


def check(wl, x, w, eps, what, **kw):
    print(f"[fused rmsnorm] {what}: rows {x.shape[0]}, in {x.shape[1]}, {x.dtype}", flush=True)
    y, out = fused(wl, x, w, eps, **kw)
    assert torch.equal(y, rmsnorm_fwd(x, w, eps).cpu()), f"{what}: y differs from the RMSNorm kernel's"
    cm = cpu_meta(wl.meta)
    xs, ws = x.cpu(), w.cpu()
    As, Bs, base = [a.cpu() for a in wl.a_stacks], [b.cpu() for b in wl.b_stacks], wl.base.cpu()
    assert_tol_f64(out, apply_f64(rmsnorm_f64(xs, ws, eps), As, Bs, cm, base, wl.col_offsets), f"{what} vs float64")
    _, want = apply_kernel_numerics(xs, As, Bs, cm, base, wl.col_offsets, shrink_input=rmsnorm_shrink_input(xs, ws, eps))
    assert_ulp_close(out, want, what=f"{what} vs the fused rounding sequence")
    return y, out


def test_c4_rmsnorm_qkv(dev):
    """256 decode tokens over 128 rank-32 adapters, q|k|v [4096, 1024, 1024]."""
    wl = synthetic.decode_qkv(device=dev)
    check(wl, scaled(wl.x, 1), wl.extra["norm_weight"], wl.extra["eps"], "c4 q|k|v")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_q_shape(dev, dtype):
    wl = synthetic.decode_q(device=dev, dtype=dtype)
    check(wl, scaled(wl.x, 2), norm_weight(wl.x.shape[1], dtype, dev, 2), 1e-6, f"decode q {dtype}")


def test_halves_equal_one_call(dev):
    """phases 1 then 2 (a base GEMM would run between) give the bits of phases 3."""
    wl = synthetic.decode_qkv(device=dev, tokens=96, seed=4)
    x, w = scaled(wl.x, 3), wl.extra["norm_weight"]
    y1, o1 = fused(wl, x, w, 1e-5)
    y2, o2 = fused(wl, x, w, 1e-5, split=True)
    assert torch.equal(y1, y2) and torch.equal(o1, o2)


@pytest.mark.parametrize("in_dim", [14336, 4104, 1024])
def test_widths(dev, in_dim):
    """A width whose RMSNorm holds eight chunks a thread (14336: the fused
    norm rows hold two and stream the rest, in the same order), a last K
    chunk only partly inside the row (4104), and a narrow row."""
    g = torch.Generator().manual_seed(in_dim)
    n_slots, rows = 16, 40
    slots = torch.randint(0, 12, (rows,), generator=g).tolist()
    ranks = [16] * 12 + [0] * 4
    wl = workload("widths", dev, [1] * rows, slots, ranks, [1.5] * n_slots, in_dim, [512], 16, 60 + in_dim % 97)
    check(wl, scaled(wl.x, 5), norm_weight(in_dim, wl.x.dtype, dev, 5), 1e-5, f"in {in_dim}")


def test_multi_row_segments_and_rank0(dev):
    """Segments of several rows (entries of up to 16 rows, a slot split over
    entries), rank-0 slots whose rows still get y and keep their output."""
    lens = [3, 1, 20, 1, 5, 1, 40, 2]
    slots = [2, 0, 1, 3, 2, 4, 5, 0]
    ranks = [16, 8, 0, 16, 16, 0]
    wl = workload("segs", dev, lens, slots, ranks, [0.5, 1.0, 2.0, 1.5, 3.0, 1.0], 2048, [1024, 256], 16, 71)
    x = scaled(wl.x, 6)
    y, out = check(wl, x, norm_weight(2048, wl.x.dtype, dev, 6), 1e-5, "multi-row segments")
    starts = [sum(lens[:i]) for i in range(len(lens))]
    rank0 = [r for a, n, sl in zip(starts, lens, slots) if ranks[sl] == 0 for r in range(a, a + n)]
    assert rank0 and torch.equal(out[rank0], wl.base.cpu()[rank0])


def test_table_without_lora_still_writes_y(dev):
    """Every slot of rank 0: the plan has no entry, the norm rows still run."""
    wl = workload("no_lora", dev, [1] * 24, [i % 8 for i in range(24)], [0] * 8, [1.0] * 8, 1024, [1024], 16, 8)
    x, w = scaled(wl.x, 7), norm_weight(1024, wl.x.dtype, dev, 7)
    y, out = fused(wl, x, w, 1e-5)
    assert torch.equal(y, rmsnorm_fwd(x, w, 1e-5).cpu())
    assert torch.equal(out, wl.base.cpu())


def test_close_to_unfused(dev):
    """The unfused schedule (RMSNorm, then the grouped apply on y) differs
    only by the rounding of the MFMA inputs."""
    wl = synthetic.decode_qkv(device=dev, tokens=128, seed=9)
    x, w = scaled(wl.x, 9), wl.extra["norm_weight"]
    _, got = fused(wl, x, w, 1e-5)
    ref = wl.clone_base()
    assert apply_grouped(rmsnorm_fwd(x, w, 1e-5), wl.a_stacks, wl.b_stacks, wl.meta, ref, wl.col_offsets, mode=2)
    torch.testing.assert_close(got.double(), ref.cpu().double(), atol=2e-2, rtol=1e-2)


def test_graph_replays_follow_new_inputs(dev):
    """Captured once, replayed three times over rewritten x (with eager work
    and synchronisations between replays): each replay equals the eager call."""
    wl = synthetic.decode_qkv(device=dev, tokens=64, seed=10)
    w = wl.extra["norm_weight"]
    lws = LinkedWorkspace()
    s = torch.cuda.Stream(dev)
    x = scaled(wl.x, 10)
    y = torch.empty_like(x)
    out = wl.clone_base()
    args = lambda: (x, w, 1e-5, y, wl.a_stacks, wl.b_stacks, wl.meta, out, wl.col_offsets, lws)
    with torch.cuda.stream(s):
        assert rmsnorm_apply_grouped(*args())  # the capture stream's workspace exists before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        assert rmsnorm_apply_grouped(*args())
    for k in range(3):
        x.copy_(scaled(torch.randn(x.shape, generator=torch.Generator().manual_seed(20 + k)).to(x.dtype).to(dev),
                       30 + k))
        out.copy_(wl.base)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got_y, got_out = y.cpu(), out.cpu()
        want_y, want_out = fused(wl, x, w, 1e-5)
        assert torch.equal(got_y, want_y) and torch.equal(got_out, want_out), f"replay {k}"


def test_rejects_y_overlapping_x(dev):
    wl = synthetic.decode_q(device=dev, tokens=16, in_dim=1024, out=1024, n_slots=8, n_adapters=4, rank=16, seed=12)
    x = wl.x.clone()
    w = norm_weight(1024, x.dtype, dev, 12)
    with pytest.raises(ValueError, match="overlaps"):
        rmsnorm_apply_grouped(x, w, 1e-5, x, wl.a_stacks, wl.b_stacks, wl.meta, wl.clone_base(), wl.col_offsets)


def test_weight_of_another_dtype_is_not_taken(dev):
    wl = synthetic.decode_q(device=dev, tokens=16, in_dim=1024, out=1024, n_slots=8, n_adapters=4, rank=16, seed=13)
    w = torch.ones(1024, device=dev, dtype=torch.float32)
    assert not rmsnorm_apply_grouped(wl.x, w, 1e-5, torch.empty_like(wl.x), wl.a_stacks, wl.b_stacks, wl.meta,
                                     wl.clone_base(), wl.col_offsets)


def test_backend_rmsnorm_apply_with_base_projection(dev):
    """HipLoRABackend.rmsnorm_apply_lora_multi on a decode table: y is the
    RMSNorm's bits, base_fn writes the base projection of y between the two
    launches, and the LoRA delta of y is added on top (float64 closed form)."""
    from multi_lora_amd import HipLoRABackend

    wl = synthetic.decode_qkv(device=dev, tokens=64, seed=14)
    x, w = scaled(wl.x, 14), wl.extra["norm_weight"]
    g = torch.Generator().manual_seed(14)
    wq = (torch.randn(sum(b.shape[1] for b in wl.b_stacks), x.shape[1], generator=g) * 0.02).to(x.dtype).to(dev)
    out = torch.empty(x.shape[0], wq.shape[0], dtype=x.dtype, device=dev)
    be = HipLoRABackend()
    be.set_kernel_input_metadata(wl.meta)
    calls = []

    def base_fn(y, o):
        calls.append(1)
        torch.mm(y, wq.t(), out=o)

    y = be.rmsnorm_apply_lora_multi(x, w, 1e-5, wl.a_stacks, wl.b_stacks, out, wl.col_offsets, base_fn=base_fn)
    torch.cuda.synchronize()
    assert calls == [1]
    assert torch.equal(y.cpu(), rmsnorm_fwd(x, w, 1e-5).cpu())
    base = (y.float() @ wq.float().t()).to(x.dtype).cpu()
    cm = cpu_meta(wl.meta)
    want = apply_f64(rmsnorm_f64(x.cpu(), w.cpu(), 1e-5), [a.cpu() for a in wl.a_stacks],
                     [b.cpu() for b in wl.b_stacks], cm, base, wl.col_offsets)
    # the base GEMM's own rounding differs from the fp32 product above by a unit of bf16
    assert_tol_f64(out.cpu(), want, "backend fused call vs float64")


def test_backend_rmsnorm_apply_prefill_table_takes_the_unfused_path(dev):
    """Segments longer than the decode path takes: RMSNorm, then the segment
    apply on y, bit for bit."""
    from multi_lora_amd import HipLoRABackend

    wl = workload("prefill", dev, [40, 3, 70], [1, 0, 2], [16, 16, 16], [1.0, 2.0, 0.5], 1024, [512, 128], 16, 15)
    x, w = scaled(wl.x, 15), norm_weight(1024, wl.x.dtype, dev, 15)
    be = HipLoRABackend()
    be.set_kernel_input_metadata(wl.meta)
    got = wl.clone_base()
    y = be.rmsnorm_apply_lora_multi(x, w, 1e-5, wl.a_stacks, wl.b_stacks, got, wl.col_offsets)
    ref = wl.clone_base()
    be.apply_lora_multi(rmsnorm_fwd(x, w, 1e-5), wl.a_stacks, wl.b_stacks, ref, wl.col_offsets)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), rmsnorm_fwd(x, w, 1e-5).cpu())
    assert torch.equal(got.cpu(), ref.cpu())


def test_table_without_plan(dev):
    """A table with no host plan: each half builds the plan on the device;
    the same bits as with the table's own plan."""
    lens = [1] * 48 + [5, 3]
    g = torch.Generator().manual_seed(16)
    slots = torch.randint(0, 20, (len(lens),), generator=g).tolist()
    ranks = [16] * 18 + [0, 0]
    planned = workload("planned", dev, lens, slots, ranks, [1.0] * 20, 2048, [1024, 256, 256], 16, 16)
    bare = workload("bare", dev, lens, slots, ranks, [1.0] * 20, 2048, [1024, 256, 256], 16, 16, with_plan=False)
    x, w = scaled(planned.x, 16), norm_weight(2048, planned.x.dtype, dev, 16)
    y1, o1 = fused(planned, x, w, 1e-5)
    y2, o2 = fused(bare, x, w, 1e-5, split=True)
    assert torch.equal(y1, y2) and torch.equal(o1, o2)


@pytest.mark.parametrize("seed", range(6))
def test_random_shapes(dev, seed):
    """Seeded random decode shapes through the fused call: dtype, pool size,
    ranks (zero, partial, full), r_max, 1-4 slices of widths that are not tile
    multiples, K, and a table of short segments; y bit-identical to the
    RMSNorm kernel's, out held to float64 and to the fused rounding sequence."""
    import random

    rng = random.Random(1000 + seed)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    r_max = rng.choice([8, 16, 24, 32, 48, 64])
    n_slices = rng.randint(1, 4 if r_max <= 32 else 3)
    in_dim = 8 * rng.randint(16, 700)
    outs = [8 * rng.randint(4, 200) for _ in range(n_slices)]
    n_slots = rng.choice([3, 7, 16, 64, 300])
    ranks = [rng.choice([0, r_max, max(1, r_max // 2), rng.randint(1, r_max)]) for _ in range(n_slots)]
    ranks[rng.randrange(n_slots)] = r_max
    lens = [rng.choice([1, 1, 1, 2, 5, 16]) for _ in range(rng.randint(1, 60))]
    slots = [rng.randrange(n_slots) for _ in lens]
    scal = [0.5 + (i % 4) * 0.25 for i in range(n_slots)]
    wl = workload(f"random{seed}", dev, lens, slots, ranks, scal, in_dim, outs, r_max, 2000 + seed, dtype=dtype)
    check(wl, scaled(wl.x, 3000 + seed), norm_weight(in_dim, dtype, dev, seed), 1e-5,
          f"random {seed}: {dtype}, r_max {r_max}, {n_slices} slices, in {in_dim}, {len(lens)} segments")


@pytest.mark.parametrize("plan", ["packed", "device"])
def test_graph_replays_follow_table_rewrites(dev, plan):
    """The fused call captured once follows a segment table rewritten in
    place between replays: through write_kernel_input_metadata (which
    rebuilds the packed plan), or, for a table without a plan, through the
    device plan build captured with the call."""
    from multi_lora_amd import HipLoRABackend
    from multi_lora_amd.batch_info import BatchLoRAInfo, fill_column, write_kernel_input_metadata
    from tests.test_gpu_grouped import _packed_meta

    wl = synthetic.decode_q(device=dev, tokens=64, in_dim=2048, out=2048, n_slots=16, n_adapters=8, rank=16, seed=17)
    a, b = wl.a_stacks[0], wl.b_stacks[0]
    x, w = scaled(wl.x, 17), norm_weight(2048, wl.x.dtype, dev, 17)
    if plan == "packed":
        meta = _packed_meta(dev, wl.seg_slots, wl.slot_ranks, wl.scalings)
    else:
        meta = make_meta(wl.seg_lens, wl.seg_slots, wl.slot_ranks, wl.scalings, dev, torch.bfloat16,
                         with_plan=False)
    be = HipLoRABackend()
    be.set_kernel_input_metadata(meta)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    out = wl.clone_base()
    with torch.cuda.stream(stream):  # the capture stream's workspace exists before capture
        y0 = be.rmsnorm_apply_lora_multi(x, w, 1e-5, [a], [b], out)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        y = be.rmsnorm_apply_lora_multi(x, w, 1e-5, [a], [b], out)
    for _ in range(3):
        out.copy_(wl.base)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager) and torch.equal(y, y0)

    new_slots = [(s + 3) % 8 for s in wl.seg_slots]
    if plan == "packed":
        assert write_kernel_input_metadata(meta, BatchLoRAInfo(new_slots, wl.slot_ranks, wl.scalings), device=dev,
                                           dtype=torch.bfloat16, seq_lens=[]) is meta
    else:
        fill_column(meta.weight_indices, new_slots, 0)
    ref_meta = make_meta(wl.seg_lens, new_slots, wl.slot_ranks, wl.scalings, dev, torch.bfloat16)
    be2 = HipLoRABackend()
    be2.set_kernel_input_metadata(ref_meta)
    eager2 = wl.clone_base()
    be2.rmsnorm_apply_lora_multi(x, w, 1e-5, [a], [b], eager2)
    torch.cuda.synchronize()
    assert not torch.equal(eager2, eager)
    for _ in range(3):
        out.copy_(wl.base)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager2)
    assert be.linked_workspace.counters()[1] == 0
