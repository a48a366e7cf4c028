"""The no-allocation decode entry point (mlora_apply_grouped_static) on the GPU.

Called through the C ABI, it must give the same bits as mlora_apply_grouped
with a caller workspace, on two calls in a row, the second with a smaller
input (the static scratch keeps the first call's contents), with the plan
given and with the plan built on the device into the scratch.
"""

import ctypes
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from multi_lora_amd import _ffi, synthetic
from multi_lora_amd.kernels.lora_ops import LinkedWorkspace, _slices, apply_grouped, seg_meta
from multi_lora_amd.synthetic import make_meta
from oracle.lora_ref import apply_f64
from tests.gpu_helpers import assert_tol_f64
from tests.test_gpu_lora import cpu_meta

pytestmark = pytest.mark.gpu


def static_call(wl, meta, mode=0):
    out = wl.clone_base()
    dev = wl.x.device
    m, keep = seg_meta(meta, dev, min(a.shape[0] for a in wl.a_stacks))
    sl = _slices(wl.a_stacks, wl.b_stacks, wl.col_offsets)
    n, r_max = len(wl.a_stacks), wl.a_stacks[0].shape[1]
    rc = _ffi.lib().mlora_apply_grouped_static(
        wl.x.data_ptr(), wl.x.stride(0), wl.x.shape[0], wl.x.shape[1], sl, n, r_max, out.data_ptr(), out.stride(0),
        ctypes.byref(m), _ffi.dtype_code(wl.x.dtype), mode, 3, _ffi.stream_ptr(dev))
    _ffi.check(rc, "mlora_apply_grouped_static")
    torch.cuda.synchronize()
    del keep
    return out.cpu()


def workspace_call(wl, meta, mode=0):
    out = wl.clone_base()
    assert apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, meta, out, wl.col_offsets, LinkedWorkspace(), mode=mode)
    torch.cuda.synchronize()
    return out.cpu()


def check_against_oracle(wl, got):
    xs, As, Bs = wl.x.cpu(), [a.cpu() for a in wl.a_stacks], [b.cpu() for b in wl.b_stacks]
    assert_tol_f64(got, apply_f64(xs, As, Bs, cpu_meta(wl.meta), wl.base.cpu(), wl.col_offsets), wl.name)


def test_static_scratch_matches_caller_workspace_on_two_calls(dev):
    big = synthetic.decode_q(device=dev, tokens=128, seed=61)
    small = synthetic.decode_q(device=dev, tokens=24, in_dim=2048, out=1024, n_slots=12, n_adapters=7, rank=32,
                               seed=62)
    for wl in (big, small):
        got = static_call(wl, wl.meta)
        assert torch.equal(got, workspace_call(wl, wl.meta))
        check_against_oracle(wl, got)


def test_static_scratch_with_a_device_built_plan_and_both_schedules(dev):
    wl = synthetic.decode_qkv(device=dev, tokens=48, n_slots=32, n_adapters=20, rank=16, seed=63)
    bare = make_meta(wl.seg_lens, wl.seg_slots, wl.slot_ranks, wl.scalings, dev, torch.bfloat16, with_plan=False)
    ref = workspace_call(wl, wl.meta)
    for mode in (1, 2):
        assert torch.equal(static_call(wl, bare, mode), ref)
        assert torch.equal(static_call(wl, wl.meta, mode), ref)
    smaller = synthetic.decode_q(device=dev, tokens=9, in_dim=1024, out=512, n_slots=6, n_adapters=4, rank=16,
                                 seed=64)
    assert torch.equal(static_call(smaller, smaller.meta), workspace_call(smaller, smaller.meta))


def test_static_entry_captured_as_the_first_library_call_in_a_fresh_process():
    """The static scratch is looked up on the first call on a device; that
    call may be under graph capture.  A child process (so no earlier call has
    made the lookup) captures the static entry first, replays the graph
    three times, and compares each replay with the workspace entry point."""
    helper = Path(__file__).resolve().parent / "static_first_call_in_capture.py"
    print(f"child: {helper.name}", flush=True)
    r = subprocess.run([sys.executable, str(helper)], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "replays equal: 3" in r.stdout
