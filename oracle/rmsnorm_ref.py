"""CPU restatement of the fused RMSNorm math (test infrastructure).

* ``rmsnorm_ref``  — multi_lora/kernels/rmsnorm.py:38-45: upcast to fp32,
  ``x * rsqrt(mean(x^2) + eps) * w`` in fp32, one rounding to x.dtype.
* ``rmsnorm_hf``   — the HF module the kernel replaces
  (multi_lora/tests/test_fused_rmsnorm.py:19-32): normalise in fp32, round
  to the input dtype, then multiply by the weight in that dtype.
* ``rmsnorm_f64``  — float64 ground truth.
* ``add_rmsnorm_ref`` — the residual add and the next RMSNorm of a decoder
  layer as the unfused modules compute them (the fusion the reference
  plans, OPTIMIZATION_TODO.md T22): ``h = x + residual`` rounded to the
  storage dtype (a bf16/fp16 tensor add), then ``rmsnorm_ref(h)``.
* ``rmsnorm_shrink_input`` — what the LoRA shrink multiplies with A when the
  RMSNorm is folded into it (no counterpart in the reference, which runs
  rmsnorm_fwd, multi_lora/kernels/rmsnorm.py:48-92, and then the shrink on
  its output): ``round(x * w)`` in the storage dtype times the row's
  ``rsqrt(mean(x^2) + eps)``, in float64.  Pinned against ``rmsnorm_f64``
  (the two differ by one rounding of x * w) in tests/test_oracle_closed_forms.py.
"""

from __future__ import annotations

import torch


def rmsnorm_ref(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    h = x.detach().cpu().float()
    var = (h * h).mean(-1, keepdim=True)
    y = h * torch.rsqrt(var + eps) * w.detach().cpu().float()
    return y.to(x.dtype)


def rmsnorm_hf(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    h = x.detach().cpu().float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return w.detach().cpu().to(x.dtype) * h.to(x.dtype)


def rmsnorm_f64(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    h = x.detach().cpu().double()
    return h / torch.sqrt((h * h).mean(-1, keepdim=True) + eps) * w.detach().cpu().double()


def add_rmsnorm_ref(x: torch.Tensor, residual: torch.Tensor, w: torch.Tensor, eps: float):
    """Returns (new residual h, normalised y)."""
    h = (x.detach().cpu().float() + residual.detach().cpu().float()).to(x.dtype)
    return h, rmsnorm_ref(h, w, eps)


def rmsnorm_shrink_input(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """float64 ``round(x * w) * rsqrt(mean(x^2) + eps)`` per row (x * w in fp32, exact for 16-bit
    operands, rounded to x.dtype)."""
    h = x.detach().cpu()
    xw = (h.float() * w.detach().cpu().float()).to(x.dtype).double()
    h64 = h.double()
    return xw / torch.sqrt((h64 * h64).mean(-1, keepdim=True) + eps)
