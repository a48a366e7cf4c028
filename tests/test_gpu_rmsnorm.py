"""HIP fused RMSNorm parity against the oracle (GPU).

Shapes follow multi_lora/tests/test_fused_rmsnorm.py (hidden 128/2560,
decode (64,1,h) and prefill (64,7,h), the non-contiguous q slice of a fused
QKV output) plus the fused-QKV benchmark input (256x4096, eps 1e-5).
"""

import pytest
import torch
import torch.nn as nn

from multi_lora_amd import synthetic
from multi_lora_amd.kernels import fuse_rmsnorm, rmsnorm_fwd
from oracle.rmsnorm_ref import rmsnorm_f64, rmsnorm_hf, rmsnorm_ref
from tests.gpu_helpers import assert_ulp_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hidden", [128, 2560])
@pytest.mark.parametrize("shape", [(64, 1), (64, 7)])
def test_matches_reference(dev, hidden, shape):
    torch.manual_seed(0)
    w = torch.randn(hidden).to(dev, torch.bfloat16)
    x = torch.randn(*shape, hidden).to(dev, torch.bfloat16)
    got = rmsnorm_fwd(x, w, 1e-6)
    assert got.shape == x.shape and got.dtype == x.dtype
    torch.testing.assert_close(got.cpu(), rmsnorm_hf(x, w, 1e-6), rtol=2e-2, atol=2e-2)
    assert_ulp_close(got.cpu(), rmsnorm_ref(x, w, 1e-6), what="vs single-rounding oracle")


@pytest.mark.parametrize("batch,seq", [(64, 1), (64, 7)])
def test_non_contiguous_input(dev, batch, seq):
    torch.manual_seed(0)
    hidden = 128
    w = torch.randn(hidden).to(dev, torch.bfloat16)
    qkv = torch.randn(batch, seq, 6144).to(dev, torch.bfloat16)
    sliced = qkv[..., :4096].view(batch, seq, 32, 128)
    assert not sliced.is_contiguous()
    got = rmsnorm_fwd(sliced, w, 1e-6)
    assert got.shape == sliced.shape
    torch.testing.assert_close(got.cpu(), rmsnorm_hf(sliced.contiguous(), w, 1e-6), rtol=2e-2, atol=2e-2)
    assert_ulp_close(got.cpu(), rmsnorm_ref(sliced.contiguous(), w, 1e-6), what="sliced")


def test_fused_qkv_benchmark_input(dev):
    wl = synthetic.decode_qkv(device=dev)
    w, eps = wl.extra["norm_weight"], wl.extra["eps"]
    got = rmsnorm_fwd(wl.x, w, eps)
    torch.testing.assert_close(got.double().cpu(), rmsnorm_f64(wl.x, w, eps), atol=2e-2, rtol=1e-2)
    assert_ulp_close(got.cpu(), rmsnorm_ref(wl.x, w, eps), what="decode_qkv rmsnorm")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hidden", [100, 4096, 14336])
def test_dtypes_and_odd_widths(dev, dtype, hidden):
    g = torch.Generator().manual_seed(hidden)
    x = torch.randn(33, hidden, generator=g).to(dev, dtype)
    w = (torch.randn(hidden, generator=g) * 0.1 + 1).to(dev, torch.float32)  # weight dtype differs from x
    got = rmsnorm_fwd(x, w, 1e-5)
    want = rmsnorm_ref(x, w, 1e-5)
    if dtype == torch.float32:
        torch.testing.assert_close(got.cpu(), want, atol=1e-5, rtol=1e-5)
    else:
        assert_ulp_close(got.cpu(), want, what=f"{dtype} h={hidden}")


def test_fuse_patches_all_and_keeps_numerics(dev):
    class RefRMSNorm(nn.Module):
        def __init__(self, hidden, eps=1e-6):
            super().__init__()
            self.weight = nn.Parameter(torch.randn(hidden))
            self.variance_epsilon = eps

        def forward(self, x):
            return rmsnorm_hf(x, self.weight, self.variance_epsilon).to(x.device)

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.n1 = RefRMSNorm(2560)
            self.n2 = RefRMSNorm(128)
            self.lin = nn.Linear(8, 8)

    torch.manual_seed(0)
    model = nn.Sequential(Block(), Block()).to(dev, torch.bfloat16)
    x1 = torch.randn(16, 1, 2560, device=dev, dtype=torch.bfloat16)
    x2 = torch.randn(16, 1, 128, device=dev, dtype=torch.bfloat16)
    want1, want2 = model[0].n1(x1), model[0].n2(x2)
    assert fuse_rmsnorm(model) == 4
    torch.testing.assert_close(model[0].n1(x1), want1, rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(model[0].n2(x2), want2, rtol=2e-2, atol=2e-2)
    assert isinstance(model[0].n1.weight, nn.Parameter)
    assert isinstance(model[0].lin, nn.Linear)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,hidden", [(256, 4096), (33, 100), (7, 14336), (64, 2560)])
def test_fused_add_rmsnorm(dev, dtype, rows, hidden):
    """residual <- round(x + residual) bit-exact; y within one unit of the
    single-rounding RMSNorm of that sum."""
    from multi_lora_amd.kernels import fused_add_rmsnorm
    from oracle.rmsnorm_ref import add_rmsnorm_ref

    g = torch.Generator().manual_seed(rows + hidden)
    x = torch.randn(rows, hidden, generator=g).to(dev, dtype)
    res = (torch.randn(rows, hidden, generator=g) * 3).to(dev, dtype)
    w = (torch.randn(hidden, generator=g) * 0.1 + 1).to(dev, dtype)
    h_ref, y_ref = add_rmsnorm_ref(x, res, w, 1e-5)
    y = fused_add_rmsnorm(x, res, w, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(res.cpu(), h_ref)
    if dtype == torch.float32:
        torch.testing.assert_close(y.cpu(), y_ref, atol=1e-5, rtol=1e-5)
    else:
        assert_ulp_close(y.cpu(), y_ref, what=f"{dtype} {rows}x{hidden}")


def test_fused_add_rmsnorm_in_place_output(dev):
    """y may overwrite x (vLLM-style in-place use)."""
    from multi_lora_amd import _ffi
    from oracle.rmsnorm_ref import add_rmsnorm_ref

    g = torch.Generator().manual_seed(11)
    x = torch.randn(16, 4096, generator=g).to(dev, torch.bfloat16)
    res = torch.randn(16, 4096, generator=g).to(dev, torch.bfloat16)
    w = torch.ones(4096, device=dev, dtype=torch.bfloat16)
    h_ref, y_ref = add_rmsnorm_ref(x, res, w, 1e-6)
    rc = _ffi.lib().mlora_add_rmsnorm(x.data_ptr(), 4096, res.data_ptr(), 4096, w.data_ptr(), _ffi.MLORA_BF16,
                                      x.data_ptr(), 4096, 16, 4096, 1e-6, _ffi.MLORA_BF16, _ffi.stream_ptr(dev))
    _ffi.check(rc, "mlora_add_rmsnorm")
    torch.cuda.synchronize()
    assert torch.equal(res.cpu(), h_ref)
    assert_ulp_close(x.cpu(), y_ref, what="in place")
