"""ctypes binding of libmlora_hip.so (declared in include/mlora_hip.h).

The library is loaded after ``import torch`` so that its dependency on
``libamdhip64.so.7`` resolves to the HIP runtime torch already mapped (both
carry that SONAME): device pointers and streams then belong to one runtime.
There is no fallback: if the library is missing or fails to load, every
entry point raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmlora_hip.so"
ABI_VERSION = 6

MLORA_F32, MLORA_F16, MLORA_BF16 = 0, 1, 2
MAX_SLICES = 4

_DTYPE_CODE = {torch.float32: MLORA_F32, torch.float16: MLORA_F16, torch.bfloat16: MLORA_BF16}

# Every symbol include/mlora_hip.h declares; checked at load time.
EXPORTS = (
    "mlora_abi_version",
    "mlora_last_error",
    "mlora_shrink_workspace_bytes",
    "mlora_apply_segments_workspace_bytes",
    "mlora_apply_segments",
    "mlora_shrink",
    "mlora_expand",
    "mlora_grouped_workspace_bytes",
    "mlora_apply_grouped",
    "mlora_rmsnorm",
    "mlora_pool_scatter",
    "mlora_add_rmsnorm",
    "mlora_plan_bytes",
    "mlora_build_plan",
    "mlora_apply_grouped_static",
    "mlora_rmsnorm_apply_grouped",
)

# include/mlora_hip.h: MLORA_STATIC_SCRATCH_BYTES
STATIC_SCRATCH_BYTES = 16 << 20

# Plan layout (include/mlora_hip.h: MLORA_PLAN_*) and workspace header words
# of mlora_apply_grouped (MLORA_WS_*).
PLAN_HEADER_WORDS = 16
PLAN_ENTRY_WORDS = 32
PLAN_ROWS = 16
PLAN_ROW_WORD = 8
WS_FALLBACKS = 0
WS_WAIT_TICKS = 1
WS_PLAN_ERRORS = 2
# Pools of up to this many slots get a device-built plan (mlora_build_plan).
PLAN_BUILD_MAX_SLOTS = 2048


# Segments of at most this many rows are short in the table summary
# (mlora_seg_meta.long_segs / long_rows / short_slots).
SHORT_SEG_ROWS = 16


class SegMeta(ctypes.Structure):
    """struct mlora_seg_meta."""

    _fields_ = [
        ("seg_indptr", ctypes.c_void_p),
        ("weight_indices", ctypes.c_void_p),
        ("lora_ranks", ctypes.c_void_p),
        ("scalings", ctypes.c_void_p),
        ("bs", ctypes.c_int32),
        ("max_len", ctypes.c_int32),
        ("num_slots", ctypes.c_int32),
        ("scal_dtype", ctypes.c_int32),
        ("long_segs", ctypes.c_int32),
        ("long_rows", ctypes.c_int32),
        ("short_slots", ctypes.c_int32),
        ("plan", ctypes.c_void_p),
        ("plan_cap", ctypes.c_int32),
        ("plan_entries", ctypes.c_int32),
    ]


class Slice(ctypes.Structure):
    """struct mlora_slice."""

    _fields_ = [
        ("a", ctypes.c_void_p),
        ("a_slot_stride", ctypes.c_int64),
        ("a_row_stride", ctypes.c_int64),
        ("b", ctypes.c_void_p),
        ("b_slot_stride", ctypes.c_int64),
        ("b_row_stride", ctypes.c_int64),
        ("out_dim", ctypes.c_int32),
        ("out_col", ctypes.c_int32),
    ]


SliceArray = Slice * MAX_SLICES


class PoolKey(ctypes.Structure):
    """mlora_pool_key: one module key's slot tensors and bank offsets."""

    _fields_ = [
        ("a", ctypes.c_void_p),
        ("a_slot_stride", ctypes.c_int64),
        ("a_off", ctypes.c_int64),
        ("b", ctypes.c_void_p),
        ("b_slot_stride", ctypes.c_int64),
        ("b_row_stride", ctypes.c_int64),
        ("b_off", ctypes.c_int64),
        ("in_dim", ctypes.c_int32),
        ("out_dim", ctypes.c_int32),
    ]

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None

_vp, _i32, _i64, _sz, _f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float
_SIGNATURES = {
    "mlora_abi_version": (ctypes.c_int, []),
    "mlora_last_error": (ctypes.c_char_p, []),
    "mlora_shrink_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "mlora_apply_segments_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "mlora_apply_segments": (
        ctypes.c_int,
        [_vp, _i64, _i32, _i32, ctypes.POINTER(Slice), _i32, _i32, _vp, _i64, ctypes.POINTER(SegMeta), _i32, _vp,
         _sz, _vp],
    ),
    "mlora_grouped_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "mlora_apply_grouped": (
        ctypes.c_int,
        [_vp, _i64, _i32, _i32, ctypes.POINTER(Slice), _i32, _i32, _vp, _i64, ctypes.POINTER(SegMeta), _i32, _vp,
         _sz, _i32, _i32, _vp],
    ),
    "mlora_shrink": (
        ctypes.c_int,
        [_vp, _i64, _i32, _i32, ctypes.POINTER(Slice), _i32, _i32, _i32, _vp, _i64, ctypes.POINTER(SegMeta), _i32, _vp,
         _sz, _vp],
    ),
    "mlora_expand": (
        ctypes.c_int,
        [_vp, _i64, _i32, ctypes.POINTER(Slice), _i32, _i32, _vp, _i64, ctypes.POINTER(SegMeta), _i32, _vp],
    ),
    "mlora_rmsnorm": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i64, _vp, _i32, _vp, _i64, _i64, _i32, _f32, _i32, _vp],
    ),
    "mlora_pool_scatter": (
        ctypes.c_int,
        [_vp, _i64, _i32, _vp, _vp, _i32, _i32, _i32, _i64, _i32, _vp],
    ),
    "mlora_add_rmsnorm": (
        ctypes.c_int,
        [_vp, _i64, _vp, _i64, _vp, _i32, _vp, _i64, _i64, _i32, _f32, _i32, _vp],
    ),
    "mlora_plan_bytes": (_sz, [_i32]),
    "mlora_apply_grouped_static": (
        ctypes.c_int,
        [_vp, _i64, _i32, _i32, ctypes.POINTER(Slice), _i32, _i32, _vp, _i64, ctypes.POINTER(SegMeta), _i32, _i32,
         _i32, _vp],
    ),
    "mlora_build_plan": (ctypes.c_int, [ctypes.POINTER(SegMeta), _i32, _vp, _i32, _vp]),
    "mlora_rmsnorm_apply_grouped": (
        ctypes.c_int,
        [_vp, _i64, _i32, _i32, _vp, _f32, _vp, _i64, ctypes.POINTER(Slice), _i32, _i32, _vp, _i64,
         ctypes.POINTER(SegMeta), _i32, _vp, _sz, _i32, _vp],
    ),
}


class MloraError(RuntimeError):
    """A launch-level failure reported by libmlora_hip (a hipError_t)."""


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m multi_lora_amd.build` "
                "(the HIP path has no CPU fallback)"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        version = handle.mlora_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libmlora_hip ABI {version} != expected {ABI_VERSION}; rebuild")
        _lib = handle
    return _lib


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def check(rc: int, what: str) -> None:
    """Map a library return code to the reference's exception types."""
    if rc == 0:
        return
    msg = lib().mlora_last_error().decode(errors="replace")
    if rc < 0:
        raise ValueError(f"{what}: {msg}")
    raise MloraError(f"{what}: {msg} (hipError {rc})")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    """The current HIP stream of ``device`` as an integer handle (the raw
    getter skips building a Stream object: about 0.06 vs 1.8 us a call)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def hip_runtimes_mapped() -> list:
    """Distinct libamdhip64 files mapped in this process (expected: one)."""
    paths = set()
    try:
        with open("/proc/self/maps") as fh:
            for line in fh:
                if "libamdhip64" in line:
                    paths.add(line.split()[-1])
    except OSError:
        pass
    return sorted(paths)
