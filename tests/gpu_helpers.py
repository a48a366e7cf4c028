"""Comparison helpers shared by the GPU parity tests."""

import torch

# The tolerance the hot path is held to against a float64 ground truth for
# 16-bit storage: max-abs <= 2e-2 and rel <= 1e-2 (assert_close semantics:
# |got - want| <= atol + rtol * |want|).
ATOL_16, RTOL_16 = 2e-2, 1e-2


def ordered_bits(t: torch.Tensor) -> torch.Tensor:
    """Monotone integer image of a 16-bit float tensor (adjacent values differ by 1)."""
    assert t.dtype in (torch.bfloat16, torch.float16)
    u = t.detach().cpu().view(torch.int16).to(torch.int32) & 0xFFFF
    mag = u & 0x7FFF
    return torch.where(u >= 0x8000, -mag, mag)


def ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return (ordered_bits(a) - ordered_bits(b)).abs()


def ulp_of(t: torch.Tensor) -> torch.Tensor:
    """Spacing of the storage format at each value of ``t`` (float64)."""
    mant = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}[t.dtype]
    v = t.detach().cpu().double().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(v)) - mant)


def assert_ulp_close(got: torch.Tensor, want: torch.Tensor, max_ulp: int = 1, max_frac: float = 0.02,
                     floor: float = 2.0 ** -7, what: str = ""):
    """Element-wise within ``max_ulp`` units of ``want`` (or ``floor`` in absolute terms, which covers
    results that cancel to near zero), and at most ``max_frac`` of elements differing at all.

    ``floor`` is one unit at the magnitude of the operands (2**-7 for
    values of order 1 in bf16): a sum of order-1 terms that cancels keeps
    that absolute error even though its own units are much finer.
    """
    assert got.shape == want.shape, (got.shape, want.shape)
    g64, w64 = got.detach().cpu().double(), want.detach().cpu().double()
    if got.dtype == torch.float32:
        torch.testing.assert_close(g64, w64, atol=1e-4, rtol=1e-4, msg=what)
        return
    diff = (g64 - w64).abs()
    allowed = torch.maximum(max_ulp * ulp_of(want), torch.full_like(diff, floor))
    bad = diff > allowed
    frac = (diff > 0).double().mean().item()
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} elements beyond {max_ulp} ulp / {floor}; worst diff {float(diff.max()):.3g}")
    assert frac <= max_frac, f"{what}: {frac:.4f} of elements differ"


def assert_tol_f64(got: torch.Tensor, want64: torch.Tensor, what: str = ""):
    if got.dtype == torch.float32:
        torch.testing.assert_close(got.double().cpu(), want64, atol=1e-4, rtol=1e-4, msg=what)
    else:
        torch.testing.assert_close(got.double().cpu(), want64, atol=ATOL_16, rtol=RTOL_16, msg=what)
