"""The C ABI library loads and exports what include/mlora_hip.h declares (CPU).

No compute call is made here: argument-validation paths return before any
HIP call, so they run without a GPU.
"""

import ctypes
import re
from pathlib import Path

import pytest

from multi_lora_amd import _ffi

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions():
    names = []
    for h in HEADERS:
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(mlora_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_built():
    assert _ffi.LIB_PATH.exists(), "run `python -m multi_lora_amd.build` first"


def test_exports_every_declared_symbol():
    lib = _ffi.lib()
    declared = declared_functions()
    assert declared, "no declarations parsed"
    assert set(declared) == set(_ffi.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version_and_empty_error():
    lib = _ffi.lib()
    assert lib.mlora_abi_version() == _ffi.ABI_VERSION
    assert isinstance(lib.mlora_last_error(), bytes)


def test_single_hip_runtime_mapped():
    import torch  # noqa: F401  (torch maps its HIP runtime first)

    _ffi.lib()
    assert len(_ffi.hip_runtimes_mapped()) <= 1, _ffi.hip_runtimes_mapped()


def _meta(bs=1, max_len=1, scal_dtype=_ffi.MLORA_BF16):
    return _ffi.SegMeta(None, None, None, None, bs, max_len, 4, scal_dtype)


def test_invalid_arguments_are_rejected_before_launch():
    lib = _ffi.lib()
    sl = _ffi.SliceArray()
    m = _meta()
    # bad dtype
    rc = lib.mlora_shrink(None, 16, 4, 16, sl, 1, 8, 1, None, 8, ctypes.byref(m), 9, None, 0, None)
    assert rc < 0 and b"dtype" in lib.mlora_last_error()
    # null segment table with bs > 0
    rc = lib.mlora_shrink(None, 16, 4, 16, sl, 1, 8, 1, None, 8, ctypes.byref(m), _ffi.MLORA_BF16, None, 0, None)
    assert rc < 0 and b"null" in lib.mlora_last_error()
    # Non-null placeholder addresses: validation fails before anything is read.
    fake = _ffi.SegMeta(256, 512, 768, 1024, 1, 1, 4, _ffi.MLORA_BF16)
    # too many slices
    rc = lib.mlora_expand(None, 8, 4, sl, 5, 8, None, 16, ctypes.byref(fake), _ffi.MLORA_BF16, None)
    assert rc < 0 and b"n_slices" in lib.mlora_last_error()
    # mid row too narrow for the slices
    rc = lib.mlora_expand(None, 4, 4, sl, 1, 8, None, 16, ctypes.byref(fake), _ffi.MLORA_BF16, None)
    assert rc < 0 and b"mid row stride" in lib.mlora_last_error()
    # slice columns past the output row stride (its last row would run off the row)
    wide = _ffi.SliceArray()
    wide[0] = _ffi.Slice(1 << 20, 8 * 64, 64, 2 << 20, 16 * 8, 8, 16, 8)
    rc = lib.mlora_expand(4096, 8, 4, wide, 1, 8, 8192, 16, ctypes.byref(fake), _ffi.MLORA_BF16, None)
    assert rc < 0 and b"exceed the output row stride" in lib.mlora_last_error()
    ws = 3 << 20
    rc = lib.mlora_apply_grouped(4096, 64, 4, 64, wide, 1, 8, 8192, 16, ctypes.byref(fake), _ffi.MLORA_BF16,
                                 ws, 1 << 20, 2, 3, None)
    assert rc < 0 and b"exceed the output row stride" in lib.mlora_last_error()
    # unsupported rank width with several slices
    rc = lib.mlora_shrink(4096, 64, 4, 64, sl, 2, 256, 1, 8192, 512, ctypes.byref(fake), _ffi.MLORA_BF16, None, 0, None)
    assert rc < 0
    # rmsnorm: bad hidden
    rc = lib.mlora_rmsnorm(None, 0, 0, 1, None, 0, None, 0, 4, 0, 1e-6, 2, None)
    assert rc < 0
    # bs == 0 is a no-op success, with nothing launched
    empty = _meta(bs=0, max_len=0)
    rc = lib.mlora_shrink(None, 16, 4, 16, sl, 1, 8, 1, None, 8, ctypes.byref(empty), _ffi.MLORA_BF16, None, 0, None)
    assert rc == 0


def test_fused_rmsnorm_grouped_rejects_bad_arguments():
    """mlora_rmsnorm_apply_grouped checks its own arguments before anything
    is read or launched: placeholder addresses are never dereferenced."""
    lib = _ffi.lib()
    fake = _ffi.SegMeta(256, 512, 768, 1024, 1, 1, 4, _ffi.MLORA_BF16)
    sl = _ffi.SliceArray()
    bf = _ffi.MLORA_BF16
    x, w, y, out, ws = 1 << 20, 2 << 20, 4 << 20, 8 << 20, 16 << 20

    def call(x=x, xs=64, rows=4, k=64, w=w, y=y, ys=64, dt=bf):
        return lib.mlora_rmsnorm_apply_grouped(x, xs, rows, k, w, 1e-5, y, ys, sl, 1, 16, out, 64,
                                               ctypes.byref(fake), dt, ws, 1 << 20, 3, None)

    assert call(dt=_ffi.MLORA_F32) == -2 and b"bf16 or fp16" in lib.mlora_last_error()
    assert call(w=None) == -1 and b"null" in lib.mlora_last_error()
    assert call(ys=32) == -1 and b"below in_dim" in lib.mlora_last_error()
    assert call(x=x + 2) == -2 and b"aligned" in lib.mlora_last_error()       # x not 16-byte aligned
    assert call(xs=68) == -2 and b"aligned" in lib.mlora_last_error()         # row stride not 8 elements
    assert call(y=x + 256) == -1 and b"overlaps" in lib.mlora_last_error()    # y's rows run into x's
    # y right after x's rows: no overlap, so the checks move on to the (empty) slices
    assert call(y=x + 4 * 64 * 2) == -1 and b"slice 0: A or B is null" in lib.mlora_last_error()
    assert call(rows=0) == 0                                                   # nothing to do


def test_errors_map_to_reference_exception_types():
    with pytest.raises(ValueError):
        _ffi.lib()  # loads
        m = _meta()
        rc = _ffi.lib().mlora_expand(None, 4, 4, _ffi.SliceArray(), 1, 8, None, 16, ctypes.byref(m), _ffi.MLORA_BF16, None)
        _ffi.check(rc, "mlora_expand")


def _r256(b):
    return (b + 255) // 256 * 256


def test_grouped_workspace_sizes():
    """Workspace sizes are host arithmetic, the same for every mode: a
    256-byte header, a 64-bit flag per (entry, slice group, 256-wide K chunk)
    for up to `rows` entries, fp32 sums per (row, chunk, column), a plan of
    `rows` entries, and an fp32 rstd per row for the fused RMSNorm form; 0
    for ineligible shapes."""
    lib = _ffi.lib()
    bf = _ffi.MLORA_BF16

    def want(in_dim, r_max, n, rows):
        kc = -(-in_dim // 256)
        groups = n if n * -(-r_max // 16) > 4 else 1
        return (256 + _r256(rows * groups * kc * 8) + _r256(rows * kc * n * r_max * 4) + _r256(4 * (16 + 32 * rows))
                + 4 * rows)

    for mode in (0, 1, 2):
        assert lib.mlora_grouped_workspace_bytes(4096, 16, 1, 128, 64, bf, mode) == want(4096, 16, 1, 128) == 164864
    assert lib.mlora_grouped_workspace_bytes(4104, 16, 3, 10, 65, bf, 1) == want(4104, 16, 3, 10)
    assert lib.mlora_grouped_workspace_bytes(4096, 32, 3, 256, 256, bf, 0) == want(4096, 32, 3, 256)  # per-slice items
    assert lib.mlora_grouped_workspace_bytes(16384, 16, 1, 8, 8, bf, 1) == want(16384, 16, 1, 8)       # 64 chunks
    assert lib.mlora_grouped_workspace_bytes(16392, 16, 1, 8, 8, bf, 1) == 0                          # 65 chunks
    assert lib.mlora_grouped_workspace_bytes(4100, 16, 1, 10, 65, bf, 1) == 0                # in_dim % 8
    assert lib.mlora_grouped_workspace_bytes(4096, 16, 1, 128, 64, _ffi.MLORA_F32, 1) == 0   # fp32 not grouped
    assert lib.mlora_grouped_workspace_bytes(4096, 72, 1, 128, 64, bf, 1) == 0               # r_max > 64
    assert lib.mlora_grouped_workspace_bytes(4096, 12, 1, 128, 64, bf, 2) == 0               # r_max % 8
    assert lib.mlora_grouped_workspace_bytes(4096, 16, 1, 128, 64, bf, 3) == 0               # bad mode
    assert lib.mlora_plan_bytes(10) == 4 * (16 + 32 * 10)


def test_plan_layout_matches_the_header():
    """The plan and workspace-header constants the host uses are the ones include/mlora_hip.h defines."""
    import re
    from pathlib import Path

    from multi_lora_amd import batch_info

    text = (Path(__file__).resolve().parents[1] / "include" / "mlora_hip.h").read_text()
    defs = {k: int(v) for k, v in re.findall(r"#define (MLORA_(?:PLAN|WS)_\w+) (\d+)", text)}
    assert defs["MLORA_PLAN_HEADER_WORDS"] == _ffi.PLAN_HEADER_WORDS == batch_info.PLAN_HEADER_WORDS
    assert defs["MLORA_PLAN_ENTRY_WORDS"] == _ffi.PLAN_ENTRY_WORDS == batch_info.PLAN_ENTRY_WORDS
    assert defs["MLORA_PLAN_ROWS"] == _ffi.PLAN_ROWS == batch_info.PLAN_ROWS
    assert defs["MLORA_PLAN_ROW_WORD"] == _ffi.PLAN_ROW_WORD == batch_info.PLAN_ROW_WORD
    assert defs["MLORA_WS_FALLBACKS"] == _ffi.WS_FALLBACKS
    assert defs["MLORA_WS_WAIT_TICKS"] == _ffi.WS_WAIT_TICKS
    assert defs["MLORA_WS_PLAN_ERRORS"] == _ffi.WS_PLAN_ERRORS


def test_grouped_rejects_bad_plans_and_missing_room():
    lib = _ffi.lib()
    sl = _ffi.SliceArray()
    sl[0] = _ffi.Slice(1 << 20, 16 * 64, 64, 2 << 20, 64 * 16, 16, 64, 0)
    # a plan pointer with no capacity
    bad = _ffi.SegMeta(256, 512, 768, 1024, 4, 1, 8, _ffi.MLORA_BF16, -1, -1, -1, 4096, 0, -1)
    rc = lib.mlora_apply_grouped(4096, 64, 4, 64, sl, 1, 16, 8192, 64, ctypes.byref(bad), _ffi.MLORA_BF16,
                                 3 << 20, 1 << 20, 1, 3, None)
    assert rc < 0 and b"capacity" in lib.mlora_last_error()
    # no plan and a pool larger than the device plan builder takes
    big = _ffi.SegMeta(256, 512, 768, 1024, 4, 1, 4096, _ffi.MLORA_BF16, -1, -1, -1, None, 0, -1)
    rc = lib.mlora_apply_grouped(4096, 64, 4, 64, sl, 1, 16, 8192, 64, ctypes.byref(big), _ffi.MLORA_BF16,
                                 3 << 20, 1 << 20, 1, 3, None)
    assert rc == -2 and b"device builder" in lib.mlora_last_error()
    rc = lib.mlora_build_plan(ctypes.byref(big), 4, 4096, 8, None)
    assert rc == -2
    # workspace too small
    ok = _ffi.SegMeta(256, 512, 768, 1024, 4, 1, 8, _ffi.MLORA_BF16, -1, -1, -1, 4096, 8, 1)
    rc = lib.mlora_apply_grouped(4096, 64, 4, 64, sl, 1, 16, 8192, 64, ctypes.byref(ok), _ffi.MLORA_BF16,
                                 3 << 20, 16, 1, 3, None)
    assert rc == -3


def test_pool_key_struct_layout():
    """mlora_pool_key as the header lays it out: 7 eight-byte fields, then two int32."""
    assert ctypes.sizeof(_ffi.PoolKey) == 64
    assert _ffi.PoolKey.in_dim.offset == 56 and _ffi.PoolKey.out_dim.offset == 60
    assert _ffi.PoolKey.b.offset == 24 and _ffi.PoolKey.b_off.offset == 48


def test_pool_scatter_rejects_bad_arguments():
    lib = _ffi.lib()
    assert lib.mlora_pool_scatter(None, 16, 1, None, None, 1, 0, 4, 16, _ffi.MLORA_BF16, None) < 0   # rank 0
    assert lib.mlora_pool_scatter(None, 16, 1, None, None, 1, 2, 4, 16, 7, None) < 0                 # dtype
    assert lib.mlora_pool_scatter(None, 16, 1, None, None, 1, 2, 4, 16, _ffi.MLORA_BF16, None) < 0   # null stage
    assert lib.mlora_pool_scatter(None, 16, 0, None, None, 1, 2, 4, 16, _ffi.MLORA_BF16, None) == 0  # nothing to do


def test_static_grouped_rejects_shapes_beyond_its_scratch():
    """The no-allocation entry point refuses a shape whose workspace exceeds
    its static scratch, before any HIP call, and the header's limit is the
    one the binding knows."""
    text = (ROOT / "include" / "mlora_hip.h").read_text()
    m = re.search(r"#define MLORA_STATIC_SCRATCH_BYTES \((\d+) << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == _ffi.STATIC_SCRATCH_BYTES
    lib = _ffi.lib()
    sl = _ffi.SliceArray()
    meta = _ffi.SegMeta(256, 512, 768, 1024, 4, 1, 8, _ffi.MLORA_BF16, -1, -1, -1, None, 0, -1)
    need = lib.mlora_grouped_workspace_bytes(16384, 64, 3, 4096, 8, _ffi.MLORA_BF16, 0)
    assert need > _ffi.STATIC_SCRATCH_BYTES
    rc = lib.mlora_apply_grouped_static(4096, 16384, 4096, 16384, sl, 3, 64, 8192, 16384, ctypes.byref(meta),
                                        _ffi.MLORA_BF16, 0, 3, None)
    assert rc == -3 and b"static scratch" in lib.mlora_last_error()


def test_scatter_stage_export_mirrors_the_reference():
    """multi_lora_amd.kernels exports scatter_stage with the reference's
    signature (multi_lora/kernels/scatter_bank.py:68), and, like every
    product entry point, has no CPU path."""
    import inspect

    import torch

    from multi_lora_amd import kernels

    assert "scatter_stage" in kernels.__all__
    params = list(inspect.signature(kernels.scatter_stage).parameters)
    assert params == ["stage", "slots", "tables", "total", "h", "rank", "BLOCK"]
    assert inspect.signature(kernels.scatter_stage).parameters["BLOCK"].default == 8192
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        kernels.scatter_stage(torch.zeros(1, 8), torch.zeros(1, dtype=torch.int64), {}, 8, 1, 1)


def test_calibration_library_exports():
    """The measurement library (built beside the product) carries the
    timeline readers and the calibration kernels; the product carries none
    of them."""
    import ctypes

    from multi_lora_amd.build import CALIB_LIB

    if not CALIB_LIB.exists():
        pytest.skip("measurement library not built")
    cal = ctypes.CDLL(str(CALIB_LIB))
    for name in ("mlora_tl_words", "mlora_tl_clear", "mlora_tl_read", "mlora_calib_empty", "mlora_calib_stream",
                 "mlora_apply_grouped"):
        assert hasattr(cal, name), name
    prod = _ffi.lib()
    for name in ("mlora_tl_words", "mlora_tl_clear", "mlora_calib_empty"):
        assert not hasattr(prod, name), name
