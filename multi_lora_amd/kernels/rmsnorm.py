"""Fused RMSNorm on the HIP kernel; same entry points as the reference.

``rmsnorm_fwd(x, weight, eps)`` follows multi_lora/kernels/rmsnorm.py:48-92:
rows are addressed with a two-level stride when ``x`` is a batch of dense
blocks (the q/k column slices of a fused QKV output), otherwise a contiguous
copy is normalised; the output is newly allocated and contiguous.
``fuse_rmsnorm(model)`` rebinds the forward of every ``*RMSNorm`` module
that has ``weight`` and ``variance_epsilon`` (rmsnorm.py:95-115).
"""

from __future__ import annotations

import torch

from .. import _ffi


def rmsnorm_fwd(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``x * rsqrt(mean(x^2, -1) + eps) * weight`` in fp32, rounded once to x.dtype."""
    if x.device.type != "cuda":
        raise RuntimeError(f"x must be on a ROCm GPU (got {x.device}); the HIP path has no CPU fallback")
    hidden = x.shape[-1]
    if weight.numel() != hidden:
        raise ValueError(f"weight has {weight.numel()} entries, hidden size is {hidden}")
    rows = x.numel() // hidden if hidden else 0
    if rows == 0:
        return torch.empty_like(x, memory_format=torch.contiguous_format)
    src = x
    if x.is_contiguous():
        outer_stride, inner_stride, inner = 0, hidden, max(rows, 1)
    elif x.dim() >= 2 and x[0].is_contiguous() and x.stride(-1) == 1:
        # Dense, equally spaced blocks (decode q/k slices of a fused QKV
        # output): inside a block rows are `hidden` apart.
        inner = max(rows // x.shape[0], 1)
        outer_stride, inner_stride = x.stride(0), hidden
    else:
        src = x.contiguous()
        outer_stride, inner_stride, inner = 0, hidden, max(rows, 1)
    w = weight.contiguous()
    if w.device != x.device:
        raise ValueError(f"weight on {w.device}, x on {x.device}")
    out = torch.empty((rows, hidden), dtype=x.dtype, device=x.device)
    rc = _ffi.lib().mlora_rmsnorm(
        src.data_ptr(), outer_stride, inner_stride, inner, w.data_ptr(), _ffi.dtype_code(w.dtype),
        out.data_ptr(), hidden, rows, hidden, float(eps), _ffi.dtype_code(x.dtype), _ffi.stream_ptr(x.device),
    )
    _ffi.check(rc, "mlora_rmsnorm")
    return out.reshape(x.shape)


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``residual += x`` (rounded to the dtype, in place), then RMSNorm of it.

    The residual add and the following RMSNorm of a decoder layer in one
    pass, the fusion the reference plans as ``fused_add_rms_norm``
    (OPTIMIZATION_TODO.md T22).  Returns the normalised rows (a new tensor);
    ``residual`` holds ``x + residual`` afterwards.
    """
    if x.device.type != "cuda":
        raise RuntimeError(f"x must be on a ROCm GPU (got {x.device}); the HIP path has no CPU fallback")
    hidden = x.shape[-1]
    if residual.shape != x.shape or residual.dtype != x.dtype or residual.device != x.device:
        raise ValueError(f"residual {tuple(residual.shape)} {residual.dtype} must match x {tuple(x.shape)} {x.dtype}")
    if weight.numel() != hidden:
        raise ValueError(f"weight has {weight.numel()} entries, hidden size is {hidden}")
    if not residual.is_contiguous():
        raise ValueError("residual must be contiguous (it is updated in place)")
    src = x.contiguous()
    rows = src.numel() // hidden if hidden else 0
    out = torch.empty((rows, hidden), dtype=x.dtype, device=x.device)
    if rows == 0:
        return out.reshape(x.shape)
    w = weight.contiguous()
    rc = _ffi.lib().mlora_add_rmsnorm(
        src.data_ptr(), hidden, residual.data_ptr(), hidden, w.data_ptr(), _ffi.dtype_code(w.dtype), out.data_ptr(),
        hidden, rows, hidden, float(eps), _ffi.dtype_code(x.dtype), _ffi.stream_ptr(x.device),
    )
    _ffi.check(rc, "mlora_add_rmsnorm")
    return out.reshape(x.shape)


def fuse_rmsnorm(model: torch.nn.Module) -> int:
    """Route every ``*RMSNorm`` module's forward through ``rmsnorm_fwd``; returns the count.

    Only the instance's ``forward`` is rebound (and, for a module that has
    one, its ``add_forward(delta, residual)`` -- residual add then norm --
    through ``fused_add_rmsnorm``): parameters, the module tree and
    ``state_dict`` are unchanged.
    """
    count = 0
    for module in model.modules():
        if not type(module).__name__.endswith("RMSNorm"):
            continue
        eps = getattr(module, "variance_epsilon", None)
        weight = getattr(module, "weight", None)
        if eps is None or weight is None:
            continue
        module.forward = _bound_forward(weight, float(eps))
        if callable(getattr(module, "add_forward", None)):
            module.add_forward = _bound_add_forward(weight, float(eps))
        count += 1
    return count


def _bound_forward(weight: torch.Tensor, eps: float):
    def forward(hidden_states: torch.Tensor) -> torch.Tensor:
        return rmsnorm_fwd(hidden_states, weight, eps)

    return forward


def _bound_add_forward(weight: torch.Tensor, eps: float):
    def add_forward(delta: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        return fused_add_rmsnorm(delta, residual, weight, eps)

    return add_forward
