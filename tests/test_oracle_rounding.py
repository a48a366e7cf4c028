"""Pins of the oracle's rounding sequences (CPU).

The constructed cases (tests/rounding_cases.py) have exact, hand-derived
results in which each rounding step changes the stored value.  The oracle
must reproduce them bit for bit, and every mutant of the oracle that drops,
moves or re-types one rounding must fail at least one of them.  Mutants are
planted in copies of the oracle's own source, so the checks test the code
that the GPU tests compare against.
"""

import inspect
import textwrap

import pytest
import torch

import oracle.lora_ref as lora_ref
import oracle.rmsnorm_ref as rmsnorm_ref_mod
from multi_lora_amd.synthetic import make_meta
from oracle.lora_ref import TorchLoRABackend, apply_kernel_numerics
from oracle.rmsnorm_ref import add_rmsnorm_ref, rmsnorm_hf, rmsnorm_ref
from tests.rounding_cases import (ADD_H, ADD_RES, ADD_X, ADD_Y, RMS_HF, RMS_ONCE, RMS_W, RMS_X, lora_cases,
                                  lora_tensors, tile)

DTYPES = [torch.bfloat16, torch.float16]


def _meta(case):
    return make_meta([1], [0], [2], [case.scale], "cpu", torch.float32)


def _kernel_numerics(fn, case, dtype):
    x, a, b, base = lora_tensors(case, dtype)
    return fn(x, [a], [b], _meta(case), base)


def _torch_backend(cls, case, dtype):
    x, a, b, base = lora_tensors(case, dtype)
    be = cls()
    be.set_kernel_input_metadata(_meta(case))
    mid = be.run_lora_a_sgemm(x, a)
    return mid, be.run_lora_b_sgemm(mid, b, base.clone())


@pytest.mark.parametrize("dtype", DTYPES)
def test_kernel_numerics_constructed_cases(dtype):
    for case in lora_cases(dtype):
        mid, out = _kernel_numerics(apply_kernel_numerics, case, dtype)
        assert mid.dtype == dtype and out.dtype == dtype
        assert mid[0, :2].double().tolist() == case.mid, case.name
        assert out.double().item() == case.kernel_out, case.name


@pytest.mark.parametrize("dtype", DTYPES)
def test_torch_backend_constructed_cases(dtype):
    for case in lora_cases(dtype):
        mid, out = _torch_backend(TorchLoRABackend, case, dtype)
        assert mid[0, :2].double().tolist() == case.mid, case.name
        assert out.double().item() == case.torch_out, case.name


def test_the_two_orders_differ_where_the_scaling_is_not_a_power_of_two():
    """Only the scaled cases separate the kernels' order from the PyTorch backend's."""
    for dtype in DTYPES:
        differ = [c.name for c in lora_cases(dtype) if c.kernel_out != c.torch_out]
        assert differ == ["scale_after_rounding", "scaling_kept_in_fp32"]


def test_rmsnorm_constructed_cases():
    x, w = tile(RMS_X, 4, torch.bfloat16), torch.full((4,), RMS_W).bfloat16()
    assert rmsnorm_hf(x, w, 0.0)[0].double().tolist() == RMS_HF
    assert rmsnorm_ref(x, w, 0.0)[0].double().tolist() == RMS_ONCE
    # the same rows repeated keep the mean of squares, so wider rows give the same values
    x64 = tile(RMS_X, 64, torch.bfloat16)
    assert rmsnorm_ref(x64, torch.full((64,), RMS_W).bfloat16(), 0.0)[0].double().tolist() == RMS_ONCE * 16


def test_add_rmsnorm_constructed_case():
    x, res = tile(ADD_X, 4, torch.bfloat16), tile(ADD_RES, 4, torch.bfloat16)
    assert torch.equal(res.float(), torch.tensor([ADD_RES])), "residual must be exact in bf16"
    h, y = add_rmsnorm_ref(x, res, torch.full((4,), 7.0).bfloat16(), 0.0)
    assert h[0].double().tolist() == ADD_H
    assert y[0].double().tolist() == ADD_Y


# ---------------------------------------------------------------- mutants
def _mutate(fn, old: str, new: str):
    """A copy of ``fn`` (a module-level function or a method) with ``old`` replaced by ``new`` in its source."""
    src = textwrap.dedent(inspect.getsource(fn))
    assert src.count(old) == 1, f"mutation site {old!r} not found once in {fn.__qualname__}"
    ns = dict(vars(inspect.getmodule(fn)))
    exec(compile(src.replace(old, new), f"<mutant of {fn.__qualname__}>", "exec"), ns)
    return ns[fn.__name__]


KERNEL_MUTANTS = {
    "mid not rounded": ("y = _round(y.float(), dt)", "y = y.float()"),
    "mid rounded to the other 16-bit format":
        ("y = _round(y.float(), dt)", "y = _round(y.float(), torch.float16 if dt == torch.bfloat16 else torch.bfloat16)"),
    "delta not rounded": ("d = _round(d, dt)", "d = d"),
    "rounded before the scaling": (".float() * scale", ".float().to(dt).float() * scale"),
    "residual scaled with the delta": ("+ d, dt)", "* scale + d, dt)"),
    "residual not added": ("_round(out[start:end, c0 : c0 + b.shape[1]] + d, dt)", "_round(d, dt)"),
}


@pytest.mark.parametrize("name", sorted(KERNEL_MUTANTS))
def test_kernel_numerics_mutants_fail_a_constructed_case(name):
    mutant = _mutate(apply_kernel_numerics, *KERNEL_MUTANTS[name])
    caught = []
    for dtype in DTYPES:
        for case in lora_cases(dtype):
            mid, out = _kernel_numerics(mutant, case, dtype)
            if mid[0, :2].double().tolist() != case.mid or out.double().item() != case.kernel_out:
                caught.append((dtype, case.name))
    assert caught, f"mutant '{name}' passes every constructed case"


TORCH_BACKEND_MUTANTS = {
    "delta in fp32, one rounding": (
        "delta = (x[start:end, :r] @ b.T) * scale",
        "delta = ((x[start:end, :r].float() @ b.float().T) * scale.float()).to(x.dtype)"),
    "scaling left in fp32": ("scale = scal[slot].to(dtype=x.dtype)", "scale = scal[slot].float()"),
    "mid without the rank cut": ("a = weights[slot, :r, :].to(dtype=x.dtype)", "a = weights[slot, :2, :].to(dtype=x.dtype) * 0"),
}


@pytest.mark.parametrize("name", sorted(TORCH_BACKEND_MUTANTS))
def test_torch_backend_mutants_fail_a_constructed_case(name):
    method = "run_lora_a_sgemm" if "mid" in name else "run_lora_b_sgemm"
    mutated = _mutate(getattr(TorchLoRABackend, method), *TORCH_BACKEND_MUTANTS[name])
    cls = type("Mutant", (TorchLoRABackend,), {method: mutated})
    caught = []
    for dtype in DTYPES:
        for case in lora_cases(dtype):
            mid, out = _torch_backend(cls, case, dtype)
            if mid[0, :2].double().tolist() != case.mid or out.double().item() != case.torch_out:
                caught.append((dtype, case.name))
    assert caught, f"mutant '{name}' passes every constructed case"


HF_MUTANTS = {
    "h not rounded before the weight": (
        "return w.detach().cpu().to(x.dtype) * h.to(x.dtype)", "return (w.detach().cpu().float() * h).to(x.dtype)"),
    "inverse rms rounded": (
        "torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)",
        "torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps).to(x.dtype).float()"),
    "mean of squares in the storage dtype": (
        "h.pow(2).mean(-1, keepdim=True)", "x.detach().cpu().pow(2).mean(-1, keepdim=True).float()"),
}

REF_MUTANTS = {
    "h rounded before the weight": (
        "y = h * torch.rsqrt(var + eps) * w.detach().cpu().float()",
        "y = (h * torch.rsqrt(var + eps)).to(x.dtype).float() * w.detach().cpu().float()"),
    "mean of squares in the storage dtype": (
        "var = (h * h).mean(-1, keepdim=True)", "var = (x.detach().cpu() * x.detach().cpu()).mean(-1, keepdim=True).float()"),
}

ADD_MUTANTS = {
    "sum normalised before rounding": (
        "return h, rmsnorm_ref(h, w, eps)",
        "return h, rmsnorm_ref(x.detach().cpu().float() + residual.detach().cpu().float(), w, eps).to(x.dtype)"),
}


@pytest.mark.parametrize("name", sorted(HF_MUTANTS))
def test_rmsnorm_hf_mutants_fail_the_constructed_case(name):
    mutant = _mutate(rmsnorm_hf, *HF_MUTANTS[name])
    x, w = tile(RMS_X, 4, torch.bfloat16), torch.full((4,), RMS_W).bfloat16()
    assert mutant(x, w, 0.0)[0].double().tolist() != RMS_HF


@pytest.mark.parametrize("name", sorted(REF_MUTANTS))
def test_rmsnorm_ref_mutants_fail_the_constructed_case(name):
    mutant = _mutate(rmsnorm_ref, *REF_MUTANTS[name])
    x, w = tile(RMS_X, 4, torch.bfloat16), torch.full((4,), RMS_W).bfloat16()
    assert mutant(x, w, 0.0)[0].double().tolist() != RMS_ONCE


@pytest.mark.parametrize("name", sorted(ADD_MUTANTS))
def test_add_rmsnorm_mutants_fail_the_constructed_case(name):
    mutant = _mutate(add_rmsnorm_ref, *ADD_MUTANTS[name])
    x, res = tile(ADD_X, 4, torch.bfloat16), tile(ADD_RES, 4, torch.bfloat16)
    h, y = mutant(x, res, torch.full((4,), 7.0).bfloat16(), 0.0)
    assert h[0].double().tolist() != ADD_H or y[0].double().tolist() != ADD_Y


def test_mutation_sites_are_live():
    """Each mutation changes the function's source (guards against a site that no longer exists)."""
    for fn, table in ((apply_kernel_numerics, KERNEL_MUTANTS), (rmsnorm_hf, HF_MUTANTS), (rmsnorm_ref, REF_MUTANTS),
                      (add_rmsnorm_ref, ADD_MUTANTS)):
        for old, _ in table.values():
            assert inspect.getsource(fn).count(old) == 1
    assert lora_ref.apply_kernel_numerics is apply_kernel_numerics
    assert rmsnorm_ref_mod.rmsnorm_hf is rmsnorm_hf
