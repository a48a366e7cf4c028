"""Run as a child process by tests/test_zz_no_alloc.py (a fresh process, so
the library's static scratch has not been looked up yet): the first call of
mlora_apply_grouped_static is made while a stream is being captured into a
HIP graph.  The graph is replayed three times, with eager work and
synchronisations between replays, and every replay is compared with the
caller-workspace entry point run eagerly afterwards.  Prints one line:
"replays equal: N" on success."""

import ctypes
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

from multi_lora_amd import _ffi, synthetic  # noqa: E402
from multi_lora_amd.kernels.lora_ops import LinkedWorkspace, _slices, apply_grouped, seg_meta  # noqa: E402


def main() -> int:
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    wl = synthetic.decode_q(device=dev, tokens=64, in_dim=1024, out=1024, n_slots=16, n_adapters=9, rank=16, seed=71)
    out = wl.clone_base()
    m, keep = seg_meta(wl.meta, dev, wl.a_stacks[0].shape[0])
    sl = _slices(wl.a_stacks, wl.b_stacks, wl.col_offsets)
    lib = _ffi.lib()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        rc = lib.mlora_apply_grouped_static(
            wl.x.data_ptr(), wl.x.stride(0), wl.x.shape[0], wl.x.shape[1], sl, 1, wl.a_stacks[0].shape[1],
            out.data_ptr(), out.stride(0), ctypes.byref(m), _ffi.dtype_code(wl.x.dtype), 0, 3, _ffi.stream_ptr(dev))
    _ffi.check(rc, "mlora_apply_grouped_static under capture")
    ref = wl.clone_base()
    assert apply_grouped(wl.x, wl.a_stacks, wl.b_stacks, wl.meta, ref, wl.col_offsets, LinkedWorkspace(), mode=0)
    torch.cuda.synchronize()
    equal = 0
    for _ in range(3):
        out.copy_(wl.base)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        equal += int(torch.equal(out, ref))
        _ = (wl.x.float() * 2).sum().item()  # eager work between replays
    del keep
    print(f"replays equal: {equal}", flush=True)
    return 0 if equal == 3 else 1


if __name__ == "__main__":
    sys.exit(main())
