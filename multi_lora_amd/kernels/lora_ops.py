"""Host entry points of the HIP segment-LoRA kernels.

Same names, argument meaning and asserts as the reference's kernel entry
points, so its kernel-level tests read the same:

* ``sgemm_lora_a_fwd(x, weights, meta, output, stack_num=1)`` —
  multi_lora/kernels/sgemm_lora_a.py:186-274;
* ``sgemm_lora_b_fwd(x, weights, meta, base_output=None)`` —
  multi_lora/kernels/sgemm_lora_b.py:156-237.

Multi-slice forms (x read once for fused QKV / gate-up; one launch for all
slices of the output) have no reference counterpart and are additive:
``sgemm_lora_a_multi_fwd`` and ``sgemm_lora_b_multi_fwd``.

Every call launches on the current HIP stream of the tensors' device and
never synchronises.  There is no CPU path: CPU tensors raise.
"""

from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from .. import _ffi
from ..batch_info import KernelInputMetaData

_WORKSPACES: Dict[Tuple[str, int], torch.Tensor] = {}


class Workspace:
    """Caller-owned scratch (fp32 split sums), grown on demand, reused across calls.

    Sequential launches on one stream may share a workspace; launches that
    overlap on different streams need separate workspaces.
    """

    def __init__(self) -> None:
        self.buf: Optional[torch.Tensor] = None

    def get(self, nbytes: int, device: torch.device) -> Tuple[int, int]:
        if nbytes <= 0:
            return 0, 0
        if self.buf is None or self.buf.numel() < nbytes or self.buf.device != device:
            size = max(nbytes, 1 << 20)
            self.buf = torch.zeros(size, dtype=torch.uint8, device=device)
        return self.buf.data_ptr(), self.buf.numel()


class LinkedWorkspace:
    """Workspaces of the grouped (decode) path, one per stream.

    Each buffer is zero-filled on allocation and used by nothing else.  The
    single launch tags the flags its work items publish with the launch's
    dispatch id on its hardware queue, which keeps launches on one stream
    apart without ever clearing the buffer; launches on different streams
    get separate buffers.  Its header words count K chunks that a work item
    computed itself after a wait gave up, and plan errors.
    """

    def __init__(self) -> None:
        self.bufs: Dict[Tuple[torch.device, int], torch.Tensor] = {}

    def get(self, nbytes: int, device: torch.device, stream: int) -> Tuple[int, int]:
        key = (device, stream)
        buf = self.bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "the decode workspace of the capturing stream does not exist yet (or is too small): it would "
                    "be allocated and zero-filled inside the graph; run the same calls once on that stream "
                    "before capturing (torch.cuda.graph(g, stream=s) after running them on s)")
            buf = self.bufs[key] = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        return buf.data_ptr(), buf.numel()

    def counters(self) -> Tuple[int, int]:
        """(chunks computed after a wait gave up, plan errors) summed over all
        buffers (synchronises).  The first only costs time; the second means a
        table's plan did not fit the call and should stay 0."""
        fb = pe = 0
        for b in self.bufs.values():
            h = b[:16].view(torch.int32).cpu()
            fb += int(h[_ffi.WS_FALLBACKS])
            pe += int(h[_ffi.WS_PLAN_ERRORS])
        return fb, pe

    def set_wait_ticks(self, ticks: int) -> None:
        """Set the wait limit of every buffer (10 ns ticks; 0 = library default;
        negative = no wait: every expand item computes every K chunk itself)."""
        for b in self.bufs.values():
            b[4 * _ffi.WS_WAIT_TICKS:4 * _ffi.WS_WAIT_TICKS + 4].view(torch.int32).fill_(int(ticks))


# mlora_grouped_workspace_bytes is host arithmetic of its arguments alone.
_GROUPED_WS_BYTES: Dict[tuple, int] = {}


def _default_workspace(device: torch.device, linked: bool = False) -> Workspace:
    key = (device.type, device.index if device.index is not None else torch.cuda.current_device(), linked)
    ws = _WORKSPACES.get(key)
    if ws is None:
        ws = _WORKSPACES[key] = LinkedWorkspace() if linked else Workspace()
    return ws


def _require_gpu(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{what} must be on a ROCm GPU (got {t.device}); the HIP path has no CPU fallback")


def _int32(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    if t.dtype == torch.int32 and t.device == device and t.is_contiguous():
        return t
    return t.to(device=device, dtype=torch.int32).contiguous()


def seg_meta(meta: KernelInputMetaData, device: torch.device, num_slots: int) -> Tuple[_ffi.SegMeta, list]:
    """Build the C segment table; returns it and the tensors it points into.

    ``num_slots`` is the slot dimension of the stacks; slots at or past it
    (or past ``lora_ranks``) are treated as rank 0 by the kernels.
    """
    if meta is None:
        raise RuntimeError("kernel_input_metadata not set; call set_kernel_input_metadata first")
    bs = int(meta.bs)
    indptr = _int32(meta.seg_indptr, device)
    widx = _int32(meta.weight_indices, device)
    ranks = _int32(meta.lora_ranks, device)
    scal = meta.scalings
    if scal.dtype not in (torch.float32, torch.float16, torch.bfloat16) or scal.device != device:
        scal = scal.to(device=device, dtype=torch.float32)
    scal = scal.contiguous()
    if indptr.numel() < bs + 1 or widx.numel() < bs:
        raise ValueError(f"metadata holds {widx.numel()} segments / {indptr.numel()} offsets for bs={bs}")
    if scal.numel() < ranks.numel():
        raise ValueError(f"scalings ({scal.numel()}) shorter than lora_ranks ({ranks.numel()})")
    n_slots = min(ranks.numel(), int(num_slots))
    summary = getattr(meta, "table_summary", None)
    long_segs, long_rows, short_slots = summary(n_slots) if summary is not None else (-1, -1, -1)
    plan = getattr(meta, "plan", None)
    if plan is not None and (plan.device != device or plan.dtype != torch.int32):
        plan = None
    m = _ffi.SegMeta(
        indptr.data_ptr(),
        widx.data_ptr(),
        ranks.data_ptr(),
        scal.data_ptr(),
        bs,
        int(meta.max_len),
        n_slots,
        _ffi.dtype_code(scal.dtype),
        long_segs,
        long_rows,
        short_slots,
        plan.data_ptr() if plan is not None else None,
        int(meta.plan_cap) if plan is not None else 0,
        int(meta.plan_entries) if plan is not None else -1,
    )
    return m, [indptr, widx, ranks, scal, plan]


def _slices(a_stacks: Sequence[Optional[torch.Tensor]], b_stacks: Sequence[Optional[torch.Tensor]],
            out_cols: Sequence[int]) -> _ffi.SliceArray:
    arr = _ffi.SliceArray()
    for i, (a, b) in enumerate(zip(a_stacks, b_stacks)):
        s = arr[i]
        if a is not None:
            s.a, s.a_slot_stride, s.a_row_stride = a.data_ptr(), a.stride(0), a.stride(1)
        if b is not None:
            s.b, s.b_slot_stride, s.b_row_stride = b.data_ptr(), b.stride(0), b.stride(1)
            s.out_dim = b.shape[1]
        s.out_col = int(out_cols[i])
    return arr


def _check_stack(w: torch.Tensor, what: str, dtype: torch.dtype, device: torch.device) -> None:
    if w.dim() != 3:
        raise ValueError(f"{what} must be 3-D [slots, rows, cols], got {tuple(w.shape)}")
    if w.stride(2) != 1:
        raise ValueError(f"{what} innermost dimension must be contiguous")
    if w.dtype != dtype or w.device != device:
        raise ValueError(f"{what} is {w.dtype} on {w.device}; expected {dtype} on {device}")


def shrink(x: torch.Tensor, a_stacks: Sequence[torch.Tensor], meta: KernelInputMetaData, output: torch.Tensor,
           *, stack_num: int = 1, workspace: Optional[Workspace] = None) -> torch.Tensor:
    """``output[t, s*r_max + n] = x[t] . A_s[slot(t), n]`` for every slice ``s``."""
    _require_gpu(x, "x")
    dev = x.device
    n = len(a_stacks)
    if not 1 <= n <= _ffi.MAX_SLICES:
        raise ValueError(f"1..{_ffi.MAX_SLICES} A stacks expected, got {n}")
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be a 2-D [S, in] tensor with contiguous rows")
    in_dim = x.shape[1]
    r_max = a_stacks[0].shape[1]
    for i, a in enumerate(a_stacks):
        _check_stack(a, f"A[{i}]", x.dtype, dev)
        if a.shape[1] != r_max or a.shape[2] != in_dim:
            raise ValueError(f"A[{i}] {tuple(a.shape)} does not match r_max={r_max}, in={in_dim}")
    if output.dim() != 2 or output.stride(1) != 1 or output.dtype != x.dtype or output.device != dev:
        raise ValueError("output must be a 2-D row-contiguous tensor of x's dtype and device")
    if output.shape[0] < x.shape[0] or output.shape[1] < n * r_max:
        raise ValueError(f"output {tuple(output.shape)} smaller than [{x.shape[0]}, {n * r_max}]")
    m, keep = seg_meta(meta, dev, min(a.shape[0] for a in a_stacks))
    lib = _ffi.lib()
    dt = _ffi.dtype_code(x.dtype)
    ws = workspace or _default_workspace(dev)
    need = lib.mlora_shrink_workspace_bytes(in_dim, r_max, n, x.shape[0], m.bs, m.max_len, dt)
    ws_ptr, ws_bytes = ws.get(need, dev)
    sl = _slices(a_stacks, [None] * n, [0] * n)
    rc = lib.mlora_shrink(
        x.data_ptr(), x.stride(0), x.shape[0], in_dim, sl, n, r_max, int(stack_num), output.data_ptr(), output.stride(0),
        ctypes.byref(m), dt, ws_ptr, ws_bytes, _ffi.stream_ptr(dev),
    )
    _ffi.check(rc, "mlora_shrink")
    del keep
    return output


def expand(mid: torch.Tensor, b_stacks: Sequence[torch.Tensor], meta: KernelInputMetaData, out: torch.Tensor,
           out_cols: Sequence[int]) -> torch.Tensor:
    """``out[t, out_cols[s] + n] += scaling * mid[t, s*r_max:(s*r_max+rank)] . B_s[slot(t), n, :rank]``."""
    _require_gpu(mid, "mid")
    dev = mid.device
    n = len(b_stacks)
    if not 1 <= n <= _ffi.MAX_SLICES:
        raise ValueError(f"1..{_ffi.MAX_SLICES} B stacks expected, got {n}")
    if mid.dim() != 2 or mid.stride(1) != 1:
        raise ValueError("mid must be a 2-D [S, n*r_max] tensor with contiguous rows")
    r_max = b_stacks[0].shape[2]
    for i, b in enumerate(b_stacks):
        _check_stack(b, f"B[{i}]", mid.dtype, dev)
        if b.shape[2] != r_max:
            raise ValueError(f"B[{i}] {tuple(b.shape)} does not match r_max={r_max}")
        if out_cols[i] < 0 or out_cols[i] + b.shape[1] > out.shape[1]:
            raise ValueError(f"slice {i}: columns [{out_cols[i]}, {out_cols[i] + b.shape[1]}) outside output "
                             f"of width {out.shape[1]}")
    if mid.shape[1] < n * r_max:
        raise ValueError(f"mid has {mid.shape[1]} columns, need {n * r_max}")
    if out.dim() != 2 or out.stride(1) != 1 or out.dtype != mid.dtype or out.device != dev:
        raise ValueError("output must be a 2-D row-contiguous tensor of mid's dtype and device")
    if out.shape[0] < mid.shape[0]:
        raise ValueError(f"output has {out.shape[0]} rows, mid has {mid.shape[0]}")
    m, keep = seg_meta(meta, dev, min(b.shape[0] for b in b_stacks))
    sl = _slices([None] * n, b_stacks, out_cols)
    rc = _ffi.lib().mlora_expand(
        mid.data_ptr(), mid.stride(0), mid.shape[0], sl, n, r_max, out.data_ptr(), out.stride(0), ctypes.byref(m),
        _ffi.dtype_code(mid.dtype), _ffi.stream_ptr(dev),
    )
    _ffi.check(rc, "mlora_expand")
    del keep
    return out


GROUPED_MAX_LEN = 16


class _DevicePlan:
    """A plan built on the device for a table that carries none, kept with the
    table while its tensors stay the same objects at the same versions."""

    __slots__ = ("key", "plan", "cap", "count_host", "ready")

    def __init__(self, key, plan, cap, count_host, ready):
        self.key, self.plan, self.cap, self.count_host, self.ready = key, plan, cap, count_host, ready


def _table_key(meta: KernelInputMetaData, rows: int, num_slots: int):
    """Identity of a table's contents as torch tracks them: each column's
    object, address and in-place version counter; None when torch does not
    track versions (inference tensors)."""
    cols = (meta.seg_indptr, meta.weight_indices, meta.lora_ranks, meta.scalings)
    try:
        return (int(meta.bs), int(rows), int(num_slots)) + tuple((id(t), t.data_ptr(), t._version) for t in cols)
    except RuntimeError:
        return None


def _device_plan(meta: KernelInputMetaData, m: "_ffi.SegMeta", rows: int, dev: torch.device) -> None:
    """Give a plan-less table a plan built on the device once, outside graph
    capture, and reuse it while the table is unchanged (torch bumps a
    tensor's version on every in-place write).  The entry count is copied to
    pinned host memory without a wait and sizes the grid once it has
    arrived.  Under capture, or for tables whose versions torch does not
    track, the library builds the plan into the workspace for every call,
    so a replayed graph follows in-place rewrites."""
    if m.num_slots > _ffi.PLAN_BUILD_MAX_SLOTS or torch.cuda.is_current_stream_capturing():
        return
    key = _table_key(meta, rows, m.num_slots)
    if key is None:
        return
    cached = getattr(meta, "_device_plan", None)
    if cached is None or cached.key != key:
        lib = _ffi.lib()
        cap = max(1, int(rows))
        plan = torch.empty(lib.mlora_plan_bytes(cap) // 4, dtype=torch.int32, device=dev)
        built = _ffi.SegMeta.from_buffer_copy(m)
        built.plan, built.plan_cap, built.plan_entries = None, 0, -1
        _ffi.check(lib.mlora_build_plan(ctypes.byref(built), int(rows), plan.data_ptr(), cap, _ffi.stream_ptr(dev)),
                   "mlora_build_plan")
        count_host = torch.empty(1, dtype=torch.int32, pin_memory=True)
        count_host.copy_(plan[:1], non_blocking=True)
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream(dev))
        cached = _DevicePlan(key, plan, cap, count_host, ready)
        meta._device_plan = cached
    m.plan, m.plan_cap = cached.plan.data_ptr(), cached.cap
    m.plan_entries = int(cached.count_host[0]) if cached.ready.query() else -1


def apply_grouped(x: torch.Tensor, a_stacks: Sequence[torch.Tensor], b_stacks: Sequence[torch.Tensor],
                  meta: KernelInputMetaData, out: torch.Tensor, out_cols: Sequence[int],
                  workspace: Optional[LinkedWorkspace] = None, phases: int = 3, mode: int = 0) -> bool:
    """Slot-grouped shrink+expand into ``out``; returns False (nothing launched) if the shape is not eligible.

    Work follows the table's plan (``meta.plan``; built on the device when
    the table has none).  ``mode`` 1 = single launch, 2 = two launches,
    0 = the library's choice (the single launch while its work items fit on
    the chip about at once); all give bit-identical results.  With two launches, ``phases`` 1 / 2 run only the shrink /
    expand half; 3 runs both.  ``workspace`` holds one buffer per stream.
    """
    _require_gpu(x, "x")
    dev = x.device
    n = len(a_stacks)
    if len(b_stacks) != n or not 1 <= n <= _ffi.MAX_SLICES:
        raise ValueError("need matching A and B stacks (1..4 slices)")
    if mode not in (0, 1, 2):
        raise ValueError(f"mode {mode} not in 0..2")
    if x.dim() != 2 or x.stride(1) != 1 or out.dim() != 2 or out.stride(1) != 1:
        return False
    in_dim, r_max = x.shape[1], a_stacks[0].shape[1]
    for i, (a, b) in enumerate(zip(a_stacks, b_stacks)):
        _check_stack(a, f"A[{i}]", x.dtype, dev)
        _check_stack(b, f"B[{i}]", x.dtype, dev)
        if a.shape[1] != r_max or a.shape[2] != in_dim or b.shape[2] != r_max:
            raise ValueError(f"slice {i}: A {tuple(a.shape)} / B {tuple(b.shape)} do not match r_max={r_max}, in={in_dim}")
        if out_cols[i] < 0 or out_cols[i] + b.shape[1] > out.shape[1]:
            raise ValueError(f"slice {i}: columns outside the output")
    if out.shape[0] < x.shape[0] or out.dtype != x.dtype or out.device != dev:
        raise ValueError("output must cover x's rows with x's dtype and device")
    lib = _ffi.lib()
    dt = _ffi.dtype_code(x.dtype)
    m, keep = seg_meta(meta, dev, min(min(a.shape[0] for a in a_stacks), min(b.shape[0] for b in b_stacks)))
    if m.plan is None:
        _device_plan(meta, m, x.shape[0], dev)
    key = (in_dim, r_max, n, x.shape[0], m.num_slots, dt, int(mode))
    need = _GROUPED_WS_BYTES.get(key)
    if need is None:
        if len(_GROUPED_WS_BYTES) >= 4096:  # row counts vary per step: keep the cache bounded
            _GROUPED_WS_BYTES.clear()
        need = _GROUPED_WS_BYTES[key] = lib.mlora_grouped_workspace_bytes(*key)
    if need == 0:
        return False
    stream = _ffi.stream_ptr(dev)
    ws_ptr, ws_bytes = (workspace or _default_workspace(dev, linked=True)).get(need, dev, stream or 0)
    sl = _slices(a_stacks, b_stacks, out_cols)
    rc = lib.mlora_apply_grouped(
        x.data_ptr(), x.stride(0), x.shape[0], in_dim, sl, n, r_max, out.data_ptr(), out.stride(0), ctypes.byref(m),
        dt, ws_ptr, ws_bytes, int(mode), int(phases), stream,
    )
    del keep
    if rc == -2:
        return False
    _ffi.check(rc, "mlora_apply_grouped")
    return True


def rmsnorm_apply_grouped(x: torch.Tensor, weight: torch.Tensor, eps: float, y: torch.Tensor,
                          a_stacks: Sequence[torch.Tensor], b_stacks: Sequence[torch.Tensor],
                          meta: KernelInputMetaData, out: torch.Tensor, out_cols: Sequence[int],
                          workspace: Optional[LinkedWorkspace] = None, phases: int = 3) -> bool:
    """RMSNorm of ``x`` into ``y`` folded into the slot-grouped apply of LoRA on ``y`` into ``out``.

    Two launches.  The first (``phases`` 1) writes ``y`` (the same bits as
    ``rmsnorm_fwd``) and the LoRA shrink, which reads ``x`` itself:
    ``round(x * weight)`` on MFMA, each row's ``rsqrt(mean(x^2) + eps)``
    applied to its sums.  The second (``phases`` 2) runs the expand into
    ``out``; a layer runs its base GEMM on ``y`` in between.  Returns False
    (nothing launched) when the call is not eligible (then run ``rmsnorm_fwd``
    and ``apply_grouped``): the grouped path's shapes, bf16/fp16, a weight of
    x's dtype, 16-byte aligned rows.  ``y`` must not overlap ``x``.  In fp16,
    ``x * weight`` must be finite in fp16 for every element.
    """
    _require_gpu(x, "x")
    dev = x.device
    n = len(a_stacks)
    if len(b_stacks) != n or not 1 <= n <= _ffi.MAX_SLICES:
        raise ValueError("need matching A and B stacks (1..4 slices)")
    if phases not in (1, 2, 3):
        raise ValueError(f"phases {phases} not in 1..3")
    if x.dim() != 2 or x.stride(1) != 1 or out.dim() != 2 or out.stride(1) != 1:
        return False
    if x.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != x.dtype or weight.dim() != 1:
        return False
    if y.dim() != 2 or y.stride(1) != 1 or y.shape != x.shape or y.dtype != x.dtype or y.device != dev:
        raise ValueError("y must be a row-contiguous tensor of x's shape, dtype and device")
    in_dim, r_max = x.shape[1], a_stacks[0].shape[1]
    if weight.shape[0] != in_dim or weight.stride(0) != 1 or weight.device != dev:
        raise ValueError(f"weight must be a contiguous [{in_dim}] tensor on x's device")
    for i, (a, b) in enumerate(zip(a_stacks, b_stacks)):
        _check_stack(a, f"A[{i}]", x.dtype, dev)
        _check_stack(b, f"B[{i}]", x.dtype, dev)
        if a.shape[1] != r_max or a.shape[2] != in_dim or b.shape[2] != r_max:
            raise ValueError(f"slice {i}: A {tuple(a.shape)} / B {tuple(b.shape)} do not match r_max={r_max}, in={in_dim}")
        if out_cols[i] < 0 or out_cols[i] + b.shape[1] > out.shape[1]:
            raise ValueError(f"slice {i}: columns outside the output")
    if out.shape[0] < x.shape[0] or out.dtype != x.dtype or out.device != dev:
        raise ValueError("output must cover x's rows with x's dtype and device")
    lib = _ffi.lib()
    dt = _ffi.dtype_code(x.dtype)
    m, keep = seg_meta(meta, dev, min(min(a.shape[0] for a in a_stacks), min(b.shape[0] for b in b_stacks)))
    if m.plan is None:
        _device_plan(meta, m, x.shape[0], dev)
    key = (in_dim, r_max, n, x.shape[0], m.num_slots, dt, 2)
    need = _GROUPED_WS_BYTES.get(key)
    if need is None:
        if len(_GROUPED_WS_BYTES) >= 4096:
            _GROUPED_WS_BYTES.clear()
        need = _GROUPED_WS_BYTES[key] = lib.mlora_grouped_workspace_bytes(*key)
    if need == 0:
        return False
    stream = _ffi.stream_ptr(dev)
    ws_ptr, ws_bytes = (workspace or _default_workspace(dev, linked=True)).get(need, dev, stream or 0)
    sl = _slices(a_stacks, b_stacks, out_cols)
    rc = lib.mlora_rmsnorm_apply_grouped(
        x.data_ptr(), x.stride(0), x.shape[0], in_dim, weight.data_ptr(), float(eps), y.data_ptr(), y.stride(0), sl,
        n, r_max, out.data_ptr(), out.stride(0), ctypes.byref(m), dt, ws_ptr, ws_bytes, int(phases), stream,
    )
    del keep
    if rc == -2:
        return False
    _ffi.check(rc, "mlora_rmsnorm_apply_grouped")
    return True


def build_plan_device(meta: KernelInputMetaData, num_rows: int, num_slots: int, cap: Optional[int] = None) -> torch.Tensor:
    """The table's plan built on the device (``mlora_build_plan``) into a new int32 tensor."""
    dev = meta.seg_indptr.device
    _require_gpu(meta.seg_indptr, "metadata")
    cap = int(num_rows) if cap is None else int(cap)
    lib = _ffi.lib()
    words = lib.mlora_plan_bytes(max(cap, 1)) // 4
    plan = torch.zeros(words, dtype=torch.int32, device=dev)
    m, keep = seg_meta(meta, dev, num_slots)
    m.plan, m.plan_cap, m.plan_entries = None, 0, -1
    rc = lib.mlora_build_plan(ctypes.byref(m), int(num_rows), plan.data_ptr(), max(cap, 1), _ffi.stream_ptr(dev))
    _ffi.check(rc, "mlora_build_plan")
    del keep
    return plan


def apply_segments(x: torch.Tensor, a_stacks: Sequence[torch.Tensor], b_stacks: Sequence[torch.Tensor],
                   meta: KernelInputMetaData, out: torch.Tensor, out_cols: Sequence[int],
                   workspace: Optional[Workspace] = None) -> torch.Tensor:
    """Segment shrink then expand into ``out`` (in place), one library call.

    Same results as ``shrink`` followed by ``expand`` element for element;
    the rank-r intermediate lives in the workspace, and where the shrink's
    reduction is split over workgroups the expand adds the split sums up
    itself (no reduce launch).
    """
    _require_gpu(x, "x")
    dev = x.device
    n = len(a_stacks)
    if len(b_stacks) != n or not 1 <= n <= _ffi.MAX_SLICES:
        raise ValueError(f"need matching A and B stacks (1..{_ffi.MAX_SLICES} slices)")
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be a 2-D [S, in] tensor with contiguous rows")
    if out.dim() != 2 or out.stride(1) != 1 or out.dtype != x.dtype or out.device != dev or out.shape[0] < x.shape[0]:
        raise ValueError("output must be a 2-D row-contiguous tensor covering x's rows, with x's dtype and device")
    in_dim, r_max = x.shape[1], a_stacks[0].shape[1]
    for i, (a, b) in enumerate(zip(a_stacks, b_stacks)):
        _check_stack(a, f"A[{i}]", x.dtype, dev)
        _check_stack(b, f"B[{i}]", x.dtype, dev)
        if a.shape[1] != r_max or a.shape[2] != in_dim or b.shape[2] != r_max:
            raise ValueError(f"slice {i}: A {tuple(a.shape)} / B {tuple(b.shape)} do not match r_max={r_max}, in={in_dim}")
        if out_cols[i] < 0 or out_cols[i] + b.shape[1] > out.shape[1]:
            raise ValueError(f"slice {i}: columns outside the output")
    m, keep = seg_meta(meta, dev, min(min(a.shape[0] for a in a_stacks), min(b.shape[0] for b in b_stacks)))
    lib = _ffi.lib()
    dt = _ffi.dtype_code(x.dtype)
    need = lib.mlora_apply_segments_workspace_bytes(in_dim, r_max, n, x.shape[0], m.bs, m.max_len, dt)
    ws_ptr, ws_bytes = (workspace or _default_workspace(dev)).get(need, dev)
    sl = _slices(a_stacks, b_stacks, out_cols)
    rc = lib.mlora_apply_segments(
        x.data_ptr(), x.stride(0), x.shape[0], in_dim, sl, n, r_max, out.data_ptr(), out.stride(0), ctypes.byref(m),
        dt, ws_ptr, ws_bytes, _ffi.stream_ptr(dev),
    )
    _ffi.check(rc, "mlora_apply_segments")
    del keep
    return out


def sgemm_lora_a_fwd(x: torch.Tensor, weights: torch.Tensor, kernel_input_metadata: KernelInputMetaData,
                     output: torch.Tensor, stack_num: int = 1) -> torch.Tensor:
    """LoRA A segment GEMM: ``output[:S, :r_max]`` = per-segment ``x @ A[slot, :r].T``.

    x: ``[S, in]``, weights: ``[K, r_max, in]``, output: a caller-owned
    ``[>=S, >=r_max]`` buffer; returns the ``[S, r_max]`` view written.
    """
    assert x.is_contiguous()
    assert weights.is_contiguous()
    assert len(x.shape) == 2
    assert len(weights.shape) == 3
    assert x.shape[-1] == weights.shape[-1]
    rows, r_max = x.shape[0], weights.shape[-2]
    out = output[:rows, :r_max]
    shrink(x, [weights], kernel_input_metadata, out, stack_num=stack_num)
    return out


def sgemm_lora_b_fwd(x: torch.Tensor, weights: torch.Tensor, kernel_input_metadata: KernelInputMetaData,
                     base_output: Optional[torch.Tensor] = None) -> torch.Tensor:
    """LoRA B segment GEMM with fused residual: ``base_output += scaling * (mid @ B[slot, :, :r].T)``.

    x (mid): ``[S, r_max]``, weights: ``[K, out, r_max]``.  With
    ``base_output=None`` a zero output is allocated and returned.
    """
    assert x.is_contiguous()
    assert weights.is_contiguous()
    assert len(x.shape) == 2
    assert len(weights.shape) == 3
    assert x.shape[-1] == weights.shape[-1]
    rows, out_dim = x.shape[0], weights.shape[-2]
    if base_output is None:
        base_output = torch.zeros((rows, out_dim), device=x.device, dtype=x.dtype)
    if base_output.dim() != 2 or base_output.shape[1] != out_dim:
        raise ValueError(f"base_output {tuple(base_output.shape)} is not [S, {out_dim}]")
    expand(x, [weights], kernel_input_metadata, base_output, [0])
    return base_output


def sgemm_lora_a_multi_fwd(x: torch.Tensor, weights: List[torch.Tensor], kernel_input_metadata: KernelInputMetaData,
                           output: torch.Tensor) -> torch.Tensor:
    """Shrink for several slices at once; returns ``output[:S, :n*r_max]`` (slice s at columns s*r_max)."""
    rows, r_max = x.shape[0], weights[0].shape[-2]
    out = output[:rows, : len(weights) * r_max]
    shrink(x.contiguous(), [w.contiguous() for w in weights], kernel_input_metadata, out)
    return out


def sgemm_lora_b_multi_fwd(x: torch.Tensor, weights: List[torch.Tensor], kernel_input_metadata: KernelInputMetaData,
                           base_output: torch.Tensor, col_offsets: Optional[Sequence[int]] = None) -> torch.Tensor:
    """Expand for several slices in one launch; slice s adds into columns starting at ``col_offsets[s]``.

    ``col_offsets`` defaults to the running sum of the slices' output widths
    (the q|k|v or gate|up concatenation).
    """
    if col_offsets is None:
        col_offsets, c = [], 0
        for w in weights:
            col_offsets.append(c)
            c += w.shape[1]
    expand(x.contiguous(), [w.contiguous() for w in weights], kernel_input_metadata, base_output, list(col_offsets))
    return base_output
