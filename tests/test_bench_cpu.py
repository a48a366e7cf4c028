"""bench.py's host side on the CPU: the workload table, the algorithmic byte
counts the roofline is priced on, and the one-GPU contract."""

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from multi_lora_amd import synthetic  # noqa: E402


def test_headline_algorithmic_bytes():
    """decode q_proj 4096->4096, 128 one-token segments over 32 rank-16
    adapters: x 1 MiB + A 4 MiB + B 4 MiB + the output read and written
    (2 MiB) = 11,534,336 bytes per call."""
    wl = bench.workload_host("decode_q")
    assert synthetic.algorithmic_bytes(wl) == 1 * 2**20 + 4 * 2**20 + 4 * 2**20 + 2 * 2**20 == 11_534_336


@pytest.mark.parametrize("name", ["decode_q_resident", "c5_gate_up", "c5_qkv", "c5_o", "c5_down"])
def test_per_call_workloads_build_with_their_shapes(name):
    """Every per-call workload that bench.py names builds on the host with
    the shapes its description gives."""
    assert name in bench.OTHER_WORKLOADS
    wl = bench.workload_host(name)
    in_dim = wl.x.shape[1]
    outs = [b.shape[1] for b in wl.b_stacks]
    if name.startswith("c5_"):
        assert wl.seg_lens == [512, 512] + [1] * 64 and wl.tokens == 1088
        assert (in_dim, outs) == {"c5_gate_up": (4096, [14336, 14336]), "c5_qkv": (4096, [4096, 1024, 1024]),
                                  "c5_o": (4096, [4096]), "c5_down": (14336, [4096])}[name]
        assert name in bench.PREFILL_WORKLOADS
    else:
        # 64 resident adapters, tokens over 32 of them: the bytes count only the referenced ones.
        assert sum(r > 0 for r in wl.slot_ranks) == 64
        assert len({s for s in wl.seg_slots}) <= 32
        assert synthetic.algorithmic_bytes(wl) == 11_534_336


def test_more_than_one_gpu_is_refused():
    """The bench measures one GPU; --gpus 2 exits with status 2 and says so,
    before touching a device."""
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
