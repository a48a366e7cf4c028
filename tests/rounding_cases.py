"""Constructed inputs whose exact results are known, one per rounding step.

Each LoRA case is one token, one slot of rank 2, storage dtype with ``p``
explicit mantissa bits (bf16: 7, fp16: 10).  All sums are exact in fp32,
so the only roundings are the ones under test, and the expected values
below are derived by hand, in the comments, from round-to-nearest-even.

The reference's GPU kernels round three times
(multi_lora/kernels/sgemm_lora_a.py:109: ``mid`` stored in the storage
dtype; multi_lora/kernels/sgemm_lora_b.py:84-89: ``acc * scaling`` rounded,
then added to the residual and rounded again).  Its per-segment PyTorch
backend (multi_lora/backend/torch_backend.py:45,82-88) runs every op in the
storage dtype, so it also rounds ``mid @ B^T`` before the scaling.

The RMSNorm cases pin the HF module the fused kernel replaces
(multi_lora/tests/test_fused_rmsnorm.py:19-32: h rounded to the input dtype
before the weight), the kernel's own single rounding
(multi_lora/kernels/rmsnorm.py:38-45), and the rounded residual sum of the
fused add + RMSNorm.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List

import torch

MANTISSA = {torch.bfloat16: 7, torch.float16: 10}


@dataclass
class LoraCase:
    name: str
    x: List[float]          # the token's two non-zero inputs
    a: List[List[float]]    # A[:2, :2] of the slot
    b: List[float]          # B[o, :2], the same for every output column o
    scale: float
    base: float             # the residual, the same for every column
    mid: List[float]        # expected mid[:2] (the storage dtype's rounding of x A^T)
    kernel_out: float       # expected output, GPU kernel order
    torch_out: float        # expected output, per-segment PyTorch backend order


def lora_cases(dtype: torch.dtype) -> List[LoraCase]:
    p = MANTISSA[dtype]
    u = 2.0 ** -p  # one ulp at 1.0
    return [
        # mid: x A^T = [1 + 3u/4, 1]; 3u/4 is past half an ulp, so mid[0]
        # rounds up to 1 + u.  B = [1, -1] then exposes it: the output is
        # u with the rounding, 3u/4 without it.
        LoraCase("mid_rounded", [1.0, 0.75 * u], [[1.0, 1.0], [1.0, 0.0]], [1.0, -1.0], 1.0, 0.0,
                 [1.0 + u, 1.0], u, u),
        # delta before the residual add: residual 4096 (ulp 4096u), delta
        # = 2048u * (1 + u/4).  Rounded, delta is 2048u, a tie above 4096
        # that goes to the even 4096; unrounded, it is past the tie and
        # the sum goes up to 4096 + 4096u.
        LoraCase("delta_rounded_before_add", [2048.0 * u, 512.0 * u * u], [[1.0, 0.0], [0.0, 1.0]], [1.0, 1.0], 1.0,
                 4096.0, [2048.0 * u, 512.0 * u * u], 4096.0, 4096.0),
        # scaling: acc = 1 + 3u/4, scale 3.  Kernel: 3 + 9u/4 with ulp 2u
        # is 1.125 ulp past 3, so 3 + 2u.  PyTorch backend: acc rounds to
        # 1 + u first, 3 + 3u is a tie between 3 + 2u and 3 + 4u, and the
        # even one is 3 + 4u.
        LoraCase("scale_after_rounding", [1.0, 0.75 * u], [[1.0, 0.0], [0.0, 1.0]], [1.0, 1.0], 3.0, 0.0,
                 [1.0, 0.75 * u], 3.0 + 2.0 * u, 3.0 + 4.0 * u),
        # a scaling the storage dtype cannot hold: 1 + 3u/4.  Kernel (fp32
        # scaling): 3 * (1 + 3u/4) = 3 + 9u/4 rounds to 3 + 2u.  PyTorch
        # backend (scaling rounded to 1 + u first): 3 + 3u, the tie, goes to
        # 3 + 4u.
        LoraCase("scaling_kept_in_fp32", [3.0, 0.0], [[1.0, 0.0], [0.0, 1.0]], [1.0, 0.0], 1.0 + 0.75 * u, 0.0,
                 [3.0, 0.0], 3.0 + 2.0 * u, 3.0 + 4.0 * u),
        # the residual is added once, after the scaling: 1 + 2 * 1 = 3.
        LoraCase("residual_added_unscaled", [1.0, 0.0], [[1.0, 0.0], [0.0, 1.0]], [1.0, 0.0], 2.0, 1.0,
                 [1.0, 0.0], 3.0, 3.0),
    ]


def lora_tensors(case: LoraCase, dtype, in_dim: int = 2, out_dim: int = 1, r_max: int = 2, n_slots: int = 1):
    """x [1, in_dim], A [n_slots, r_max, in_dim], B [n_slots, out_dim, r_max], base [1, out_dim] on the CPU;
    the case sits in slot 0, every other entry is zero."""
    x = torch.zeros(1, in_dim)
    x[0, :2] = torch.tensor(case.x, dtype=torch.float64).float()
    a = torch.zeros(n_slots, r_max, in_dim)
    a[0, :2, :2] = torch.tensor(case.a)
    b = torch.zeros(n_slots, out_dim, r_max)
    b[0, :, :2] = torch.tensor(case.b)
    base = torch.full((1, out_dim), case.base)
    t = (x.to(dtype), a.to(dtype), b.to(dtype), base.to(dtype))
    for src, dst in zip((x, a, b, base), t):
        assert torch.equal(dst.float(), src), f"{case.name}: inputs must be exact in {dtype}"
    return t


# ---------------------------------------------------------------- RMSNorm
# x = [1.9921875, 1.5, 1.5, 1.0], w = 7, eps 0 (bf16): mean(x^2) = 2.36720276, r = 0.64995348.
#   HF (h rounded first): h = [1.2948, 0.9749, 0.9749, 0.6500] rounds to
#     [166, 250, 250, 166] ulps = [1.296875, 0.9765625, 0.9765625, 0.6484375];
#     times 7 = [9.078125, 6.8359375, .., 4.5390625] = [145.25, 218.75, .., 145.25] ulps
#     -> [9.0625, 6.84375, 6.84375, 4.53125].
#   One rounding: 7h = [9.0638, 6.8245, 6.8245, 4.5497] = [145.02, 218.38, .., 145.59] ulps
#     -> [9.0625, 6.8125, 6.8125, 4.5625].
#   r rounded to bf16 (166.39 -> 166 ulps of 2^-8) or mean(x^2) taken in bf16 gives
#   [9.0, 6.8125, 6.8125, 4.53125] instead.
RMS_X = [1.9921875, 1.5, 1.5, 1.0]
RMS_W = 7.0
RMS_HF = [9.0625, 6.84375, 6.84375, 4.53125]
RMS_ONCE = [9.0625, 6.8125, 6.8125, 4.5625]

# Fused add: x = 1, residual = [2^-8 + 2^-10 (three times), 2^-7 + 2^-9], w = 7, eps 0 (bf16).
#   Every sum rounds to 1 + 2^-7, a constant row, so y = w = 7 in every column.
#   Normalising the unrounded sums instead gives 7.0257 in the last column,
#   which rounds to 7.03125.
ADD_X = [1.0, 1.0, 1.0, 1.0]
ADD_RES = [2.0 ** -8 + 2.0 ** -10] * 3 + [2.0 ** -7 + 2.0 ** -9]
ADD_H = [1.0 + 2.0 ** -7] * 4
ADD_Y = [7.0, 7.0, 7.0, 7.0]


def tile(values: List[float], hidden: int, dtype) -> torch.Tensor:
    """One row of ``hidden`` columns repeating ``values`` (the mean of squares is unchanged)."""
    reps = hidden // len(values)
    assert reps * len(values) == hidden
    return torch.tensor(values * reps, dtype=torch.float32).to(dtype).reshape(1, hidden)
