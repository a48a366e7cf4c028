"""Seeded random shapes through both HIP paths, against the oracle (GPU).

Each case draws dtype, pool size, ranks (below, at, and zero), r_max,
slices and their widths, K, and a segment table, within the documented
limits of the path under test.  The decode path (segments of at most 16
rows) must match float64 to the bf16/fp16 tolerance and the kernels'
rounding sequence to one unit, with its two schedules bit-identical; the
segment path (prefill and mixed batches) the same, with the one-call path
bit-identical to shrink then expand; long reductions over long segments
(the streamed shrink's 128-row tiles) are drawn separately.
"""

import random

import pytest
import torch

from multi_lora_amd.kernels.lora_ops import LinkedWorkspace, Workspace, apply_grouped, apply_segments
from multi_lora_amd.synthetic import make_meta
from oracle.lora_ref import apply_f64, apply_kernel_numerics
from tests.gpu_helpers import assert_tol_f64, assert_ulp_close
from tests.test_gpu_lora import cpu_meta, run_hip

pytestmark = pytest.mark.gpu


def draw(rng: random.Random, decode: bool):
    dtype = rng.choice([torch.bfloat16, torch.float16])
    r_max = rng.choice([8, 16, 24, 32, 40, 48, 56, 64]) if decode else rng.choice([4, 8, 12, 16, 32, 64])
    n_slices = rng.randint(1, 4 if r_max <= 32 else 3)
    in_dim = 8 * rng.randint(8, 640)
    outs = [8 * rng.randint(4, 200) for _ in range(n_slices)]
    n_slots = rng.choice([3, 7, 16, 64, 300])
    ranks = [rng.choice([0, r_max, max(1, r_max // 2), rng.randint(1, r_max)]) for _ in range(n_slots)]
    ranks[rng.randrange(n_slots)] = r_max
    n_seg = rng.randint(1, 60 if decode else 12)
    if decode:
        lens = [rng.choice([1, 1, 1, 2, 5, 16]) for _ in range(n_seg)]
    else:
        lens = [rng.choice([1, 1, 3, 40, 97, 300]) for _ in range(n_seg)]
        if max(lens) <= 16:
            lens[0] = 70
    slots = [rng.randrange(n_slots) for _ in lens]
    return dtype, r_max, in_dim, outs, n_slots, ranks, lens, slots


def build(dev, seed, dtype, r_max, in_dim, outs, n_slots, ranks, lens, slots):
    g = torch.Generator().manual_seed(seed)
    rows = sum(lens)
    x = torch.randn(rows, in_dim, generator=g).to(dtype)
    As = [(torch.randn(n_slots, r_max, in_dim, generator=g) * in_dim ** -0.5).to(dtype) for _ in outs]
    Bs = [(torch.randn(n_slots, o, r_max, generator=g) * 0.05).to(dtype) for o in outs]
    base = torch.randn(rows, sum(outs), generator=g).to(dtype)
    cols = [sum(outs[:i]) for i in range(len(outs))]
    scal = [0.5 + (i % 4) * 0.25 for i in range(n_slots)]
    meta = make_meta(lens, slots, ranks, scal, dev, dtype)
    return x, As, Bs, base, cols, meta


def oracle_check(out, x, As, Bs, base, cols, meta, what):
    cm = cpu_meta(meta)
    assert_tol_f64(out, apply_f64(x, As, Bs, cm, base, cols), what)
    assert_ulp_close(out, apply_kernel_numerics(x, As, Bs, cm, base, cols)[1], what=what)


@pytest.mark.parametrize("seed", range(12))
def test_decode_path_random_shapes(dev, seed):
    rng = random.Random(1000 + seed)
    case = draw(rng, decode=True)
    x, As, Bs, base, cols, meta = build(dev, seed, *case)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    lws = LinkedWorkspace()
    outs = {}
    for mode in (1, 2):
        out = base.to(dev).clone()
        assert apply_grouped(xd, Ad, Bd, meta, out, cols, lws, mode=mode), f"case {seed}: {case[:5]} not eligible"
        torch.cuda.synchronize()
        outs[mode] = out.cpu()
    assert torch.equal(outs[1], outs[2]), f"case {seed}: schedules differ"
    assert lws.counters()[1] == 0
    oracle_check(outs[1], x, As, Bs, base, cols, meta, f"decode case {seed} {case[:5]}")


@pytest.mark.parametrize("seed", range(10))
def test_segment_path_random_shapes(dev, seed):
    rng = random.Random(2000 + seed)
    case = draw(rng, decode=False)
    x, As, Bs, base, cols, meta = build(dev, seed, *case)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    _, two = run_hip(xd, Ad, Bd, meta, base.to(dev), cols)
    one = base.to(dev).clone()
    apply_segments(xd, Ad, Bd, meta, one, cols, workspace=Workspace())
    torch.cuda.synchronize()
    assert torch.equal(one.cpu(), two), f"case {seed}: one call differs from shrink + expand"
    oracle_check(two, x, As, Bs, base, cols, meta, f"segment case {seed} {case[:5]}")


def draw_long_k(rng: random.Random):
    """Long reductions over long segments (K 8192..16384, at least 256 rows a
    segment on average, at most four A blocks a launch): the streamed
    shrink's 128-row tiles."""
    dtype = rng.choice([torch.bfloat16, torch.float16])
    r_max = rng.choice([16, 32, 64])
    n_slices = 1 if r_max == 64 else rng.randint(1, 2)
    in_dim = 8 * rng.randint(1024, 2048)
    outs = [8 * rng.randint(16, 160) for _ in range(n_slices)]
    n_slots = rng.choice([3, 7, 16])
    ranks = [rng.choice([0, r_max, max(1, r_max // 2), rng.randint(1, r_max)]) for _ in range(n_slots)]
    ranks[rng.randrange(n_slots)] = r_max
    lens = [rng.choice([256, 300, 520, 700, 1, 3]) for _ in range(rng.randint(1, 4))]
    if sum(lens) < 256 * len(lens):
        lens[0] = 256 * len(lens)
    slots = [rng.randrange(n_slots) for _ in lens]
    return dtype, r_max, in_dim, outs, n_slots, ranks, lens, slots


@pytest.mark.parametrize("seed", range(4))
def test_segment_path_long_k_random_shapes(dev, seed):
    case = draw_long_k(random.Random(5000 + seed))
    x, As, Bs, base, cols, meta = build(dev, seed, *case)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    _, two = run_hip(xd, Ad, Bd, meta, base.to(dev), cols)
    one = base.to(dev).clone()
    apply_segments(xd, Ad, Bd, meta, one, cols, workspace=Workspace())
    torch.cuda.synchronize()
    assert torch.equal(one.cpu(), two), f"long-K case {seed}: one call differs from shrink + expand"
    oracle_check(two, x, As, Bs, base, cols, meta, f"long-K case {seed} {case[:4]} lens {case[6]}")
