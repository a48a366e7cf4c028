"""Committed golden vectors (tests/golden/, written by make_golden.py).

The vectors were computed with plain numpy in float64, row by row, apart
from the oracle's code; the CPU tests pin the oracle (and the input
generator, by digest) to them, the GPU tests pin the HIP fp32 path.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from multi_lora_amd import synthetic

HERE = Path(__file__).resolve().parent / "golden"
STEP = 16


def lora_golden():
    return np.load(HERE / "cpu_small_lora.npz", allow_pickle=False)


def rms_golden():
    return np.load(HERE / "rmsnorm_small.npz", allow_pickle=False)


def _digest(t: torch.Tensor) -> str:
    import hashlib

    return hashlib.sha256(np.ascontiguousarray(t.numpy()).tobytes()).hexdigest()


def check_out(out: np.ndarray, g, atol: float) -> None:
    np.testing.assert_allclose(out[:, ::STEP], g["out_sample"], rtol=0, atol=atol)
    np.testing.assert_allclose(out.sum(axis=1), g["out_row_sums"], rtol=0, atol=atol * out.shape[1] ** 0.5 * 4)
    np.testing.assert_allclose(out.sum(axis=0), g["out_col_sums"], rtol=0, atol=atol * out.shape[0] ** 0.5 * 4)


def test_generator_reproduces_the_fixture_inputs():
    g = lora_golden()
    wl = synthetic.cpu_small()
    assert _digest(wl.x) == str(g["digest_x"])
    assert _digest(wl.a_stacks[0]) == str(g["digest_a"])
    assert _digest(wl.b_stacks[0]) == str(g["digest_b"])
    assert _digest(wl.base) == str(g["digest_base"])
    assert wl.seg_lens == g["seg_lens"].tolist() and wl.seg_slots == g["seg_slots"].tolist()


def test_oracle_f64_matches_golden():
    from oracle.lora_ref import apply_f64, shrink_ref

    g = lora_golden()
    wl = synthetic.cpu_small()
    out = apply_f64(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, wl.base).numpy()
    check_out(out, g, atol=1e-10)
    mid = shrink_ref(wl.x.double(), [a.double() for a in wl.a_stacks], wl.meta).numpy()
    np.testing.assert_allclose(mid, g["mid"], rtol=0, atol=1e-10)


def test_oracle_torch_backend_fp32_matches_golden():
    from oracle.lora_ref import TorchLoRABackend

    g = lora_golden()
    wl = synthetic.cpu_small()
    be = TorchLoRABackend()
    be.set_kernel_input_metadata(wl.meta)
    out = be.apply_lora(wl.x, wl.a_stacks[0], wl.b_stacks[0], wl.clone_base()).double().numpy()
    check_out(out, g, atol=2e-5)


def test_oracle_rmsnorm_matches_golden():
    from oracle.rmsnorm_ref import rmsnorm_f64, rmsnorm_ref

    g = rms_golden()
    x, w, eps = torch.from_numpy(g["x"]), torch.from_numpy(g["w"]), float(g["eps"])
    np.testing.assert_allclose(rmsnorm_f64(x, w, eps).numpy(), g["y"], rtol=0, atol=1e-12)
    np.testing.assert_allclose(rmsnorm_ref(x, w, eps).double().numpy(), g["y"], rtol=2e-6, atol=2e-6)


@pytest.mark.gpu
def test_hip_fp32_apply_matches_golden(dev):
    from multi_lora_amd import HipLoRABackend

    g = lora_golden()
    wl = synthetic.cpu_small(device=dev)
    be = HipLoRABackend()
    be.set_kernel_input_metadata(wl.meta)
    out = be.apply_lora(wl.x, wl.a_stacks[0], wl.b_stacks[0], wl.clone_base())
    torch.cuda.synchronize()
    check_out(out.double().cpu().numpy(), g, atol=2e-5)
    mid = be.run_lora_a_sgemm(wl.x, wl.a_stacks[0])
    torch.cuda.synchronize()
    np.testing.assert_allclose(mid.double().cpu().numpy(), g["mid"], rtol=0, atol=2e-5)


@pytest.mark.gpu
def test_hip_rmsnorm_fp32_matches_golden(dev):
    from multi_lora_amd.kernels.rmsnorm import rmsnorm_fwd

    g = rms_golden()
    x, w = torch.from_numpy(g["x"]).to(dev), torch.from_numpy(g["w"]).to(dev)
    y = rmsnorm_fwd(x, w, float(g["eps"]))
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.double().cpu().numpy(), g["y"], rtol=2e-6, atol=2e-6)
