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


def assert_ulp_close(got: torch.Tensor, want: torch.Tensor, max_ulp: int = 1, max_frac: float = 0.02, what: str = ""):
    """Element-wise at most ``max_ulp`` units apart, and at most ``max_frac`` of elements differing at all."""
    assert got.shape == want.shape, (got.shape, want.shape)
    if got.dtype == torch.float32:
        torch.testing.assert_close(got.cpu(), want.cpu(), atol=1e-4, rtol=1e-4, msg=what)
        return
    d = ulp_distance(got, want)
    frac = (d > 0).float().mean().item()
    assert int(d.max()) <= max_ulp, f"{what}: max ulp distance {int(d.max())} (frac differing {frac:.4f})"
    assert frac <= max_frac, f"{what}: {frac:.4f} of elements differ"


def assert_tol_f64(got: torch.Tensor, want64: torch.Tensor, what: str = ""):
    if got.dtype == torch.float32:
        torch.testing.assert_close(got.double().cpu(), want64, atol=1e-4, rtol=1e-4, msg=what)
    else:
        torch.testing.assert_close(got.double().cpu(), want64, atol=ATOL_16, rtol=RTOL_16, msg=what)
