"""Pins of the oracle's arithmetic (CPU): brute force, closed forms, invariants.

The reference ships no golden vectors for this path, so the float oracle is
pinned by checks a plausible mistake cannot pass: an explicit-loop float64
dot-product brute force, an identity-adapter case whose answer is known in
closed form, and the reference's own invariants (rank-0 and empty segments
are no-ops, grouped == row-wise, multi-slice == per-slice).  The mutation
tests at the end plant mistakes in copies of the oracle and show each pin
catches them.
"""

import math

import pytest
import torch

from multi_lora_amd.synthetic import cpu_small, make_meta
from oracle.lora_ref import TorchLoRABackend, apply_f64, apply_kernel_numerics, lora_delta, segments, shrink_ref
from oracle.rmsnorm_ref import rmsnorm_f64, rmsnorm_hf, rmsnorm_ref


def _tiny(seed=0, dtype=torch.float32, in_dim=6, out=5, r_max=4, n_slots=3, lens=(2, 0, 3, 1), slots=(1, 0, 2, 1),
          ranks=(3, 0, 2), garbage_tail=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(sum(lens), in_dim, generator=g).to(dtype)
    a = torch.randn(n_slots, r_max, in_dim, generator=g).to(dtype)
    b = torch.randn(n_slots, out, r_max, generator=g).to(dtype)
    if not garbage_tail:
        for s, r in enumerate(ranks):
            a[s, r:] = 0
            b[s, :, r:] = 0
    base = torch.randn(sum(lens), out, generator=g).to(dtype)
    scal = [0.5, 1.5, 2.0][:n_slots]
    meta = make_meta(list(lens), list(slots), list(ranks), scal, "cpu", torch.float32)
    return x, a, b, base, meta


def brute_force(x, a, b, base, lens, slots, ranks, scal):
    """Python-float loops: out[t][o] = base + s * sum_n (sum_k x[t][k] a[n][k]) * b[o][n]."""
    out = base.double().tolist()
    t0 = 0
    for n_tok, slot in zip(lens, slots):
        r = ranks[slot]
        for t in range(t0, t0 + n_tok):
            if r == 0:
                continue
            y = [sum(float(x[t, k]) * float(a[slot, n, k]) for k in range(x.shape[1])) for n in range(r)]
            for o in range(b.shape[1]):
                out[t][o] += scal[slot] * sum(y[n] * float(b[slot, o, n]) for n in range(r))
        t0 += n_tok
    return torch.tensor(out, dtype=torch.float64)


def test_apply_f64_matches_brute_force():
    lens, slots, ranks, scal = (2, 0, 3, 1), (1, 0, 2, 1), (3, 0, 2), [0.5, 1.5, 2.0]
    x, a, b, base, meta = _tiny()
    got = apply_f64(x, [a], [b], meta, base)
    want = brute_force(x, a, b, base, lens, slots, ranks, scal)
    assert torch.allclose(got, want, atol=1e-12, rtol=1e-12)


def test_torch_backend_matches_brute_force_fp32():
    lens, slots, ranks, scal = (2, 0, 3, 1), (1, 0, 2, 1), (3, 0, 2), [0.5, 1.5, 2.0]
    x, a, b, base, meta = _tiny()
    be = TorchLoRABackend()
    be.set_kernel_input_metadata(meta)
    got = be.apply_lora(x, a, b, base.clone())
    want = brute_force(x, a, b, base, lens, slots, ranks, scal)
    assert torch.allclose(got.double(), want, atol=1e-5, rtol=1e-5)


def test_identity_adapter_closed_form():
    """A = [I_r 0], B = [I_r; 0]: delta = scaling * x[:, :r] in the first r columns, 0 elsewhere."""
    in_dim, out, r_max, r = 8, 6, 4, 3
    x = torch.randn(5, in_dim, generator=torch.Generator().manual_seed(1))
    a = torch.zeros(1, r_max, in_dim)
    b = torch.zeros(1, out, r_max)
    a[0, :r, :r] = torch.eye(r)
    b[0, :r, :r] = torch.eye(r)
    a[0, r:] = 7.0  # stale rows beyond the rank must be ignored
    b[0, :, r:] = -3.0
    base = torch.zeros(5, out)
    meta = make_meta([5], [0], [r], [1.5], "cpu", torch.float32)
    want = torch.zeros(5, out, dtype=torch.float64)
    want[:, :r] = 1.5 * x[:, :r].double()
    assert torch.equal(apply_f64(x, [a], [b], meta, base), want)
    be = TorchLoRABackend()
    be.set_kernel_input_metadata(meta)
    assert torch.allclose(be.apply_lora(x, a, b, base.clone()).double(), want, atol=1e-6)
    mid, out_k = apply_kernel_numerics(x, [a], [b], meta, base)
    assert torch.allclose(out_k.double(), want, atol=1e-6)


def test_rank0_and_empty_segments_leave_base_bit_identical():
    x, a, b, base, meta = _tiny(ranks=(0, 0, 0))
    be = TorchLoRABackend()
    be.set_kernel_input_metadata(meta)
    assert torch.equal(be.apply_lora(x, a, b, base.clone()), base)
    assert torch.equal(apply_kernel_numerics(x, [a], [b], meta, base)[1], base)


def test_mid_beyond_rank_is_zero():
    x, a, b, base, meta = _tiny()
    mid = shrink_ref(x, [a], meta)
    for start, end, slot, r, _ in segments(meta):
        assert torch.count_nonzero(mid[start:end, r:]) == 0
    # rows of rank-0 segments are zero entirely (slot 0 has rank 0 -> rows 2..4? none: lens[1]=0)
    be = TorchLoRABackend()
    be.set_kernel_input_metadata(meta)
    assert torch.equal(be.run_lora_a_sgemm(x, a), mid)


def test_grouped_equals_rowwise_oracle():
    # multi_lora/tests/test_grouped_rows.py:92-165 in oracle form
    g = torch.Generator().manual_seed(0)
    in_dim, out, r_max = 96, 256, 64
    a = torch.randn(2, r_max, in_dim, generator=g) * 0.1
    b = torch.randn(2, out, r_max, generator=g) * 0.1
    for rows_per in (2, 8):
        rows = 2 * rows_per
        x = torch.randn(rows, in_dim, generator=g)
        base = torch.randn(rows, out, generator=g)
        grouped = make_meta([rows_per, rows_per], [0, 1], [8, 16], [1.0, 2.0], "cpu", torch.float32)
        rowwise = make_meta([1] * rows, [0] * rows_per + [1] * rows_per, [8, 16], [1.0, 2.0], "cpu", torch.float32)
        og = apply_f64(x, [a], [b], grouped, base)
        orow = apply_f64(x, [a], [b], rowwise, base)
        assert torch.allclose(og, orow, atol=1e-10)


def test_multi_slice_equals_per_slice():
    g = torch.Generator().manual_seed(5)
    in_dim, outs, r_max = 16, [12, 4, 4], 8
    x = torch.randn(7, in_dim, generator=g)
    a_s = [torch.randn(3, r_max, in_dim, generator=g) for _ in outs]
    b_s = [torch.randn(3, o, r_max, generator=g) for o in outs]
    base = torch.randn(7, sum(outs), generator=g)
    meta = make_meta([3, 4], [2, 0], [5, 0, 8], [1.0, 0.0, 0.5], "cpu", torch.float32)
    fused = apply_f64(x, a_s, b_s, meta, base, [0, 12, 16])
    sep = base.double().clone()
    c0 = 0
    for a, b, o in zip(a_s, b_s, outs):
        sep[:, c0:c0 + o] = apply_f64(x, [a], [b], meta, base[:, c0:c0 + o])
        c0 += o
    assert torch.allclose(fused, sep, atol=1e-12)


def test_lora_delta_closed_form():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 3, 10, generator=g)
    a = torch.randn(6, 10, generator=g)
    b = torch.randn(7, 6, generator=g)
    d = lora_delta(x, a, b, 0.25, rank=4)
    assert d.shape == (2, 3, 7)
    want = 0.25 * torch.einsum("stk,nk,on->sto", x.double(), a[:4].double(), b[:, :4].double())
    assert torch.allclose(d.double(), want, atol=1e-5)


def test_kernel_numerics_rounding_sequence_bf16():
    """bf16 storage: mid and delta are rounded once each; result within bf16 rounding of fp64."""
    wl = cpu_small(dtype=torch.bfloat16)
    mid, out = apply_kernel_numerics(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, wl.base)
    assert mid.dtype == torch.bfloat16 and out.dtype == torch.bfloat16
    ref = apply_f64(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, wl.base)
    torch.testing.assert_close(out.double(), ref, atol=2e-2, rtol=1e-2)
    # and it is not simply the base: the adapters contribute
    assert (out.float() - wl.base.float()).abs().max() > 1e-2


# ------------------------------------------------------------------ RMSNorm
def test_rmsnorm_closed_form_constant_rows():
    """Row of constant c: mean(x^2)=c^2, so y = c / sqrt(c^2 + eps) * w."""
    for c in (0.5, -3.0, 1e-3):
        x = torch.full((2, 16), c)
        w = torch.linspace(0.5, 2.0, 16)
        want = c / math.sqrt(c * c + 1e-6) * w.double()
        assert torch.allclose(rmsnorm_ref(x, w, 1e-6).double(), want.expand(2, 16), atol=1e-6)
        assert torch.allclose(rmsnorm_f64(x, w, 1e-6), want.expand(2, 16), atol=1e-12)


def test_rmsnorm_variants_agree_within_bf16():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 7, 2560, generator=g).bfloat16()
    w = torch.randn(2560, generator=g).bfloat16()
    ref = rmsnorm_ref(x, w, 1e-6)
    torch.testing.assert_close(ref.float(), rmsnorm_hf(x, w, 1e-6).float(), atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(ref.double(), rmsnorm_f64(x, w, 1e-6), atol=2e-2, rtol=1e-2)


# ------------------------------------------------------------------ mutations
def _mutant_transposed_b(x, a_stacks, b_stacks, meta, base, cols=None):
    out = base.double().clone()
    for start, end, slot, r, sc in segments(meta):
        a = a_stacks[0][slot, :r].double()
        bt = b_stacks[0][slot, :r, :].double()  # wrong: rows instead of columns
        out[start:end] += sc * (x[start:end].double() @ a.T) @ bt[:, : out.shape[1]]
    return out


def _mutant_ignores_rank(x, a_stacks, b_stacks, meta, base, cols=None):
    out = base.double().clone()
    for start, end, slot, r, sc in segments(meta):
        a = a_stacks[0][slot].double()
        b = b_stacks[0][slot].double()
        out[start:end] += sc * (x[start:end].double() @ a.T) @ b.T
    return out


def _mutant_no_scaling(x, a_stacks, b_stacks, meta, base, cols=None):
    out = base.double().clone()
    for start, end, slot, r, sc in segments(meta):
        out[start:end] += (x[start:end].double() @ a_stacks[0][slot, :r].double().T) @ b_stacks[0][slot, :, :r].double().T
    return out


def _mutant_wrong_slot(x, a_stacks, b_stacks, meta, base, cols=None):
    out = base.double().clone()
    n = a_stacks[0].shape[0]
    for start, end, slot, r, sc in segments(meta):
        s2 = (slot + 1) % n
        out[start:end] += sc * (x[start:end].double() @ a_stacks[0][s2, :r].double().T) @ b_stacks[0][s2, :, :r].double().T
    return out


@pytest.mark.parametrize("mutant", [_mutant_transposed_b, _mutant_ignores_rank, _mutant_no_scaling, _mutant_wrong_slot])
def test_pins_catch_planted_mistakes(mutant):
    """Each mutant of the oracle fails the brute-force pin (it would not go unnoticed)."""
    lens, slots, ranks, scal = (2, 0, 3, 1), (1, 0, 2, 1), (3, 0, 2), [0.5, 1.5, 2.0]
    x, a, b, base, meta = _tiny(in_dim=6, out=4, r_max=4)
    want = brute_force(x, a, b, base, lens, slots, ranks, scal)
    got = mutant(x, [a], [b], meta, base)
    assert not torch.allclose(got, want, atol=1e-6)


def test_add_rmsnorm_closed_forms():
    """A zero residual reduces to RMSNorm of x; a residual of -x gives h = 0
    and y = 0; sums of bf16 values that are exactly representable stay exact."""
    from oracle.rmsnorm_ref import add_rmsnorm_ref, rmsnorm_ref

    g = torch.Generator().manual_seed(2)
    x = torch.randn(5, 64, generator=g).bfloat16()
    w = (torch.randn(64, generator=g) * 0.1 + 1).bfloat16()
    h, y = add_rmsnorm_ref(x, torch.zeros_like(x), w, 1e-5)
    assert torch.equal(h, x) and torch.equal(y, rmsnorm_ref(x, w, 1e-5))
    h, y = add_rmsnorm_ref(x, -x, w, 1e-5)
    assert not h.any() and not y.any()
    ints = torch.randint(-64, 64, (5, 64), generator=g).bfloat16()
    h, _ = add_rmsnorm_ref(ints, ints, w, 1e-5)
    assert torch.equal(h, (2 * ints.float()).bfloat16())


# ------------------------------------------- RMSNorm folded into the shrink
def _rows_at_scales(n, k, seed, lo=-2.0, hi=2.0):
    """n rows of k N(0,1) values, row i scaled by 10**u with u uniform in [lo, hi]."""
    g = torch.Generator().manual_seed(seed)
    scale = 10.0 ** (torch.rand(n, 1, generator=g) * (hi - lo) + lo)
    return (torch.randn(n, k, generator=g) * scale).bfloat16(), g


def test_rmsnorm_shrink_input_closed_form_constant_rows():
    """Row of constant c and w = 1: round(c * 1) = c, so the input is c / sqrt(c^2 + eps)."""
    from oracle.rmsnorm_ref import rmsnorm_shrink_input

    for c in (0.5, -3.0, 1e-3, 96.0):
        x = torch.full((3, 32), c).bfloat16()
        want = float(x[0, 0]) / math.sqrt(float(x[0, 0]) ** 2 + 1e-5)
        got = rmsnorm_shrink_input(x, torch.ones(32).bfloat16(), 1e-5)
        assert torch.allclose(got, torch.full((3, 32), want, dtype=torch.float64), rtol=0, atol=1e-12)


def test_rmsnorm_shrink_input_is_rmsnorm_up_to_one_rounding():
    """Against the float64 RMSNorm, the fused shrink input differs only by the
    rounding of x * w to bf16: relative error at most 2^-8 per element, over
    rows whose scales span four decades (so a missing or misplaced rstd shows)."""
    from oracle.rmsnorm_ref import rmsnorm_f64, rmsnorm_shrink_input

    x, g = _rows_at_scales(48, 512, 7)
    w = (torch.randn(512, generator=g) * 0.3 + 2.0).bfloat16()
    got = rmsnorm_shrink_input(x, w, 1e-5)
    want = rmsnorm_f64(x, w, 1e-5)
    rel = ((got - want).abs() / want.abs().clamp_min(1e-30)).max().item()
    assert rel <= 2.0 ** -8, rel

    # Planted mistakes fail the same bound: no rstd at all, rstd taken from
    # x * w instead of x, and the mean over a wrong count (a dropped column).
    xw = (x.float() * w.float()).bfloat16().double()
    x64 = x.double()
    mutants = {
        "no rstd": xw,
        "rstd of x*w": xw / torch.sqrt((xw * xw).mean(-1, keepdim=True) + 1e-5),
        "mean over k-1": xw / torch.sqrt((x64 * x64).sum(-1, keepdim=True) / 511 + 1e-5),
    }
    for name, m in mutants.items():
        r = ((m - want).abs() / want.abs().clamp_min(1e-30)).max().item()
        assert r > 2.0 ** -8, name


def test_fused_rmsnorm_lora_numerics_match_closed_form():
    """The fused form's rounding sequence (the shrink on rmsnorm_shrink_input)
    stays within the bf16 tolerance of float64 RMSNorm followed by the LoRA
    closed form, on rows at scales over four decades."""
    from oracle.rmsnorm_ref import rmsnorm_f64, rmsnorm_shrink_input

    wl = cpu_small(dtype=torch.bfloat16)
    x, g = _rows_at_scales(wl.x.shape[0], wl.x.shape[1], 11)
    w = (torch.randn(wl.x.shape[1], generator=g) * 0.1 + 1.0).bfloat16()
    _, out = apply_kernel_numerics(x, wl.a_stacks, wl.b_stacks, wl.meta, wl.base,
                                   shrink_input=rmsnorm_shrink_input(x, w, 1e-5))
    ref = apply_f64(rmsnorm_f64(x, w, 1e-5), wl.a_stacks, wl.b_stacks, wl.meta, wl.base)
    torch.testing.assert_close(out.double(), ref, atol=2e-2, rtol=1e-2)
    # fed x itself instead, the sequence misses the closed form
    _, bad = apply_kernel_numerics(x, wl.a_stacks, wl.b_stacks, wl.meta, wl.base)
    assert not torch.allclose(bad.double(), ref, atol=2e-2, rtol=1e-2)
