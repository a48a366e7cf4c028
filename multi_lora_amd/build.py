"""Build libmlora_hip.so (gfx950) in-tree from multi_lora_amd/csrc/*.hip.

Usage: ``python -m multi_lora_amd.build`` (or ``__graft_entry__.build()``).
Each source is compiled to an object under ``multi_lora_amd/_build/`` in
parallel, then linked into ``multi_lora_amd/libmlora_hip.so``.

The same sources, compiled again with ``MLORA_TIMELINE`` (per-phase
timestamps in the planned decode kernel) and linked with
``csrc/calib/*.hip`` (an empty kernel and a streaming kernel), make
``multi_lora_amd/libmlora_calib.so``: the measurement library that
``bench.py --calibrate`` loads.  The product path never loads it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libmlora_hip.so"
CALIB_LIB = PKG / "libmlora_calib.so"
ARCH = os.environ.get("MLORA_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed fp32 ops are kept out of every kernel: the device pass must not
    # form v_pk_* fp32 arithmetic from ordinary float code.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # Leading pointer / integer kernel arguments arrive preloaded in SGPRs
    # (gfx950), so a kernel's first loads need not wait for the kernel
    # argument segment.
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; a ROCm toolchain is required to build libmlora_hip.so")
    return exe


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def calib_sources() -> list[Path]:
    return sorted((CSRC / "calib").glob("*.hip"))


def _compile(job) -> Path:
    src, obj, extra = job
    cmd = [_hipcc(), *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


def _link(objs, lib: Path) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of {lib.name} failed:\n{proc.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = True) -> Path:
    """Compile every HIP source, link the product library and the
    measurement library; returns the product library's path."""
    cal_dir = BUILD / "calib"
    cal_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = [(s, BUILD / (s.stem + ".o"), []) for s in srcs]
    cal_jobs = [(s, cal_dir / (s.stem + ".o"), ["-DMLORA_TIMELINE=1"]) for s in srcs + calib_sources()]
    workers = min(len(jobs) + len(cal_jobs), int(os.environ.get("MAX_JOBS", "8")), 16)
    with ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        objs = list(pool.map(_compile, jobs + cal_jobs))
    _link(objs[:len(jobs)], LIB)
    _link(objs[len(jobs):], CALIB_LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources and {CALIB_LIB.name}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
