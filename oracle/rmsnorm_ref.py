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
