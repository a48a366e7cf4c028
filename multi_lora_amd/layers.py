"""LoRA-wrapped linear layers (mirrors multi_lora/layers.py:13-142).

``LinearWithLoRA`` computes the base GEMM and then lets the backend add
every segment's LoRA delta into the result in place; the result may be a
strided view (a column slice of a fused QKV output) and is never copied.
``QKVProjGroup`` fuses the q/k/v base GEMMs of one attention block in decode;
when the backend offers ``apply_lora_multi`` the three LoRA deltas are also
applied by one shrink (x read once) and one three-slice expand.
"""

from __future__ import annotations

from typing import Dict, List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .backend.base import LoRABackend

# Process-wide switch: when off, wrapped layers return the base output only.
LORA_ENABLED = True


def set_lora_enabled(enabled: bool) -> None:
    global LORA_ENABLED
    LORA_ENABLED = bool(enabled)


def lora_delta(x: torch.Tensor, lora_a: torch.Tensor, lora_b: torch.Tensor, scaling: float, *, rank: int) -> torch.Tensor:
    """Closed form ``scaling * x @ A[:rank].T @ B[:, :rank].T`` (a test helper, not a kernel path)."""
    a = lora_a[:rank]
    b = lora_b[:, :rank]
    flat = x.reshape(-1, x.shape[-1])
    delta = (flat @ a.T @ b.T) * scaling
    return delta.reshape(*x.shape[:-1], b.shape[0])


class LinearWithLoRA(nn.Module):
    """``base_layer(x)`` plus the per-segment LoRA delta from the backend."""

    def __init__(self, base_layer: nn.Module) -> None:
        super().__init__()
        self.base_layer = base_layer
        self.backend: Optional[LoRABackend] = None
        self.A_buffer: Optional[torch.Tensor] = None
        self.B_buffer: Optional[torch.Tensor] = None
        self.qkv_group: Optional["QKVProjGroup"] = None
        self.qkv_slice: Optional[tuple] = None

    def set_lora_info(self, backend: LoRABackend, a_buffer: torch.Tensor, b_buffer: torch.Tensor) -> None:
        """Bind the step's backend and this module's slot stacks ``[K, r_max, in]`` / ``[K, out, r_max]``."""
        self.backend = backend
        self.A_buffer = a_buffer
        self.B_buffer = b_buffer

    def has_lora(self) -> bool:
        return LORA_ENABLED and self.backend is not None and self.A_buffer is not None and self.B_buffer is not None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.qkv_group is not None:
            return self.qkv_group.forward(self, x)
        return self.add_delta(x, self.base_layer(x))

    def add_delta(self, x: torch.Tensor, y_base: torch.Tensor) -> torch.Tensor:
        """Add the LoRA delta into ``y_base`` (possibly a strided view) and return it."""
        if not self.has_lora():
            return y_base
        x_flat = x.reshape(-1, x.shape[-1])
        y_flat = y_base.reshape(-1, y_base.shape[-1])
        y_flat = self.backend.apply_lora(x_flat, self.A_buffer, self.B_buffer, y_flat)
        return y_flat.reshape(y_base.shape)


class QKVProjGroup:
    """One base GEMM and one multi-slice LoRA call for sibling projections
    that read the same input: q/k/v of an attention block
    (multi_lora/layers.py:91-142), or gate/up of an MLP.  Bias-free.

    Decode-shaped inputs (one row per sequence) always take the fused path,
    as in the reference.  With ``all_shapes`` every input does: prefill and
    mixed batches then read x once for all slices, in one library call.
    """

    def __init__(self, wrappers: List[LinearWithLoRA], all_shapes: bool = False) -> None:
        if any(w.base_layer.bias is not None for w in wrappers):
            raise RuntimeError("QKV fusion requires bias=None")
        self.wrappers = list(wrappers)
        widths = [int(w.base_layer.weight.shape[0]) for w in wrappers]
        self.weight = torch.cat([w.base_layer.weight.detach() for w in wrappers], dim=0)
        col = 0
        for w, width in zip(wrappers, widths):
            # Each layer's weight becomes a view of the fused weight: no extra memory.
            w.base_layer.weight = nn.Parameter(self.weight[col : col + width], requires_grad=False)
            w.qkv_slice = (col, col + width)
            w.qkv_group = self
            col += width
        self._cached_x: Optional[torch.Tensor] = None
        self._cached_out: Optional[torch.Tensor] = None
        self._delta_done = False
        self.all_shapes = all_shapes

    def _multi_ready(self) -> bool:
        first = self.wrappers[0]
        return (
            all(w.has_lora() for w in self.wrappers)
            and all(w.backend is first.backend for w in self.wrappers)
            and hasattr(first.backend, "apply_lora_multi")
            and len({w.A_buffer.shape[1] for w in self.wrappers}) == 1
        )

    def forward(self, wrapper: LinearWithLoRA, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-2] != 1 and not self.all_shapes:
            return wrapper.add_delta(x, wrapper.base_layer(x))
        if self._cached_x is not x:
            self._cached_x = x
            self._cached_out = F.linear(x, self.weight)
            self._delta_done = False
            if self._multi_ready():
                first = self.wrappers[0]
                x_flat = x.reshape(-1, x.shape[-1])
                out_flat = self._cached_out.reshape(-1, self._cached_out.shape[-1])
                first.backend.apply_lora_multi(
                    x_flat,
                    [w.A_buffer for w in self.wrappers],
                    [w.B_buffer for w in self.wrappers],
                    out_flat,
                    [w.qkv_slice[0] for w in self.wrappers],
                )
                self._delta_done = True
        start, end = wrapper.qkv_slice
        y = self._cached_out[..., start:end]
        if self._delta_done:
            return y
        return wrapper.add_delta(x, y)


QKV_LEAVES = ("q_proj", "k_proj", "v_proj")
GATE_UP_LEAVES = ("gate_proj", "up_proj")


def _fuse_siblings(wrappers: Dict[str, LinearWithLoRA], leaves, all_shapes: bool) -> int:
    """Group the wrappers named ``<parent>.<leaf>`` by parent; every parent
    holding all of ``leaves`` becomes one group, in ``leaves`` order."""
    blocks: Dict[str, Dict[str, LinearWithLoRA]] = {}
    for name, wrapper in wrappers.items():
        parent, dot, leaf = name.rpartition(".")
        if dot and leaf in leaves and wrapper.qkv_group is None:
            blocks.setdefault(parent, {})[leaf] = wrapper
    complete = [block for block in blocks.values() if len(block) == len(leaves)]
    for block in complete:
        QKVProjGroup([block[leaf] for leaf in leaves], all_shapes=all_shapes)
    return len(complete)


def fuse_qkv_projections(wrappers: Dict[str, LinearWithLoRA], all_shapes: bool = False) -> int:
    """Fuse the base GEMMs of every attention block whose q, k and v
    projections are all wrapped (multi_lora/layers.py:128-142); returns the
    number of blocks fused.  Wrappers are matched by their parent module's
    name, so ``...self_attn.q_proj`` joins ``...self_attn.k_proj``."""
    return _fuse_siblings(wrappers, QKV_LEAVES, all_shapes)


def fuse_gate_up_projections(wrappers: Dict[str, LinearWithLoRA], all_shapes: bool = True) -> int:
    """The same for every MLP whose gate and up projections are both wrapped:
    one base GEMM and one two-slice LoRA call over their shared input."""
    return _fuse_siblings(wrappers, GATE_UP_LEAVES, all_shapes)
