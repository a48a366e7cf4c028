"""The HIP kernels on the constructed rounding cases (tests/rounding_cases.py).

Every value in these cases is exact in fp32 up to the roundings under test,
so the kernels must store exactly the hand-derived results, whatever their
summation order: the segment shrink and expand as two launches, the one-call
segment path, the planned decode kernel in both schedules, the RMSNorm
kernel and the fused residual add + RMSNorm.  The inputs are padded with
zeros (and the RMSNorm rows repeat their pattern) to the decode shape's
widths, so the K split and the output tiles are the production ones.
"""

import pytest
import torch

from multi_lora_amd.kernels import sgemm_lora_a_fwd, sgemm_lora_b_fwd
from multi_lora_amd.kernels.lora_ops import LinkedWorkspace, apply_grouped, apply_segments
from multi_lora_amd.kernels.rmsnorm import fused_add_rmsnorm, rmsnorm_fwd
from multi_lora_amd.synthetic import make_meta
from tests.rounding_cases import (ADD_H, ADD_RES, ADD_X, ADD_Y, RMS_ONCE, RMS_W, RMS_X, lora_cases, lora_tensors,
                                  tile)

pytestmark = pytest.mark.gpu

IN_DIM, OUT_DIM, R_MAX, SLOTS = 4096, 512, 16, 4


def _inputs(case, dtype, dev):
    x, a, b, base = lora_tensors(case, dtype, IN_DIM, OUT_DIM, R_MAX, SLOTS)
    meta = make_meta([1], [0], [2, 0, 0, 0], [case.scale] * SLOTS, dev, torch.float32)
    return x.to(dev), a.to(dev), b.to(dev), base.to(dev), meta


def _expect(out, case, what):
    want = torch.full((1, OUT_DIM), case.kernel_out, dtype=torch.float64)
    got = out.cpu().double()
    assert torch.equal(got, want), f"{what} {case.name}: got {got[0, :4].tolist()}, want {case.kernel_out}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_segment_kernels_store_the_constructed_results(dev, dtype):
    for case in lora_cases(dtype):
        x, a, b, base, meta = _inputs(case, dtype, dev)
        mid = torch.full((1, R_MAX), float("nan"), dtype=dtype, device=dev)
        out = base.clone()
        sgemm_lora_a_fwd(x, a, meta, mid)
        sgemm_lora_b_fwd(mid, b, meta, base_output=out)
        torch.cuda.synchronize()
        assert mid[0, :2].cpu().double().tolist() == case.mid, case.name
        assert not mid[0, 2:].cpu().any(), case.name
        _expect(out, case, "shrink+expand")
        out = base.clone()
        apply_segments(x, [a], [b], meta, out, [0])
        torch.cuda.synchronize()
        _expect(out, case, "apply_segments")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", [1, 2])
def test_decode_kernel_stores_the_constructed_results(dev, dtype, mode):
    ws = LinkedWorkspace()
    for case in lora_cases(dtype):
        x, a, b, base, meta = _inputs(case, dtype, dev)
        out = base.clone()
        assert apply_grouped(x, [a], [b], meta, out, [0], ws, mode=mode)
        torch.cuda.synchronize()
        _expect(out, case, f"planned decode mode {mode}")


def test_rmsnorm_kernels_store_the_constructed_results(dev):
    hidden = 4096
    x = tile(RMS_X, hidden, torch.bfloat16).to(dev)
    w = torch.full((hidden,), RMS_W, dtype=torch.bfloat16, device=dev)
    y = rmsnorm_fwd(x, w, 0.0)
    assert y.cpu().double()[0].tolist() == RMS_ONCE * (hidden // 4)
    res = tile(ADD_RES, hidden, torch.bfloat16).to(dev)
    y = fused_add_rmsnorm(tile(ADD_X, hidden, torch.bfloat16).to(dev), res, w, 0.0)
    assert res.cpu().double()[0].tolist() == ADD_H * (hidden // 4)
    assert y.cpu().double()[0].tolist() == ADD_Y * (hidden // 4)
