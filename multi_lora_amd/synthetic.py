"""Seeded synthetic segment-LoRA workloads at the benchmark shapes.

Every workload is drawn from one ``torch.Generator('cpu')`` in a fixed order
(slot assignment, segment lengths, ranks, x, A rows of the occupied slots in
slot order, B, residual), in fp32, then cast to the storage dtype and moved
to ``device``.  ``N(0, v)`` with a ``1/in`` argument is read as a variance
(std ``in**-0.5``); ``N(0, 0.02)`` is read as a standard deviation.
Occupied slots are ``0..n_adapters-1``; the other slots have rank 0.

Workloads (one per benchmark configuration):

* ``cpu_small``      fp32 1024->1024, 4 slots of rank 8, segments [5,17,42] -> slots [2,0,3].
* ``decode_q``       Llama-3-8B q_proj 4096->4096 bf16, 128 one-token segments,
                     64-slot pool holding 32 rank-16 adapters, uniform slot per token.
* ``prefill_mlp``    gate|up 4096->2x14336 (two slices) and down 14336->4096,
                     8 segments of U[64,1024] tokens, ranks from {16,32,64}, r_max 64.
* ``decode_qkv``     RMSNorm then q|k|v [4096,1024,1024] bf16, 256 one-token segments,
                     256-slot pool holding 128 rank-32 adapters.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch

from .batch_info import KernelInputMetaData, build_plan, plan_words


@dataclass
class LoRAWorkload:
    name: str
    x: torch.Tensor
    a_stacks: List[torch.Tensor]
    b_stacks: List[torch.Tensor]
    base: torch.Tensor
    meta: KernelInputMetaData
    col_offsets: List[int]
    seg_lens: List[int]
    seg_slots: List[int]
    slot_ranks: List[int]
    scalings: List[float]
    extra: dict = field(default_factory=dict)

    @property
    def tokens(self) -> int:
        return int(self.x.shape[0])

    def clone_base(self) -> torch.Tensor:
        return self.base.clone()


def make_meta(seg_lens: List[int], seg_slots: List[int], slot_ranks: List[int], scalings: List[float],
              device, scal_dtype: torch.dtype, host_copies: bool = True, with_plan: bool = True) -> KernelInputMetaData:
    """A segment table on ``device``; ``host_copies`` keeps the host lists for
    the table summary, and ``with_plan`` attaches the table's plan, as
    write_kernel_input_metadata does."""
    indptr = [0]
    for n in seg_lens:
        indptr.append(indptr[-1] + n)
    dev = torch.device(device)
    meta = KernelInputMetaData(
        bs=len(seg_lens),
        seg_lens=torch.tensor(seg_lens, dtype=torch.int32, device=dev),
        seg_indptr=torch.tensor(indptr, dtype=torch.int32, device=dev),
        weight_indices=torch.tensor(seg_slots, dtype=torch.int32, device=dev),
        lora_ranks=torch.tensor(slot_ranks, dtype=torch.int32, device=dev),
        scalings=torch.tensor(scalings, dtype=scal_dtype, device=dev),
        max_len=max(seg_lens) if seg_lens else 0,
    )
    if host_copies:
        meta.set_host_copies(seg_lens, seg_slots)
    if with_plan and dev.type == "cuda":
        attach_plan(meta, indptr, seg_slots, slot_ranks, scalings, scal_dtype)
    return meta


def attach_plan(meta: KernelInputMetaData, indptr, seg_slots, slot_ranks, scalings, scal_dtype) -> None:
    """Build the table's plan on the host and attach it (a device tensor) to ``meta``."""
    n_slots = len(slot_ranks)
    rows = int(indptr[-1]) if len(indptr) else 0
    cap = max(1, len(seg_slots) + min(len(seg_slots), n_slots))
    words = np.zeros(plan_words(cap), dtype=np.int32)
    scal_f32 = torch.tensor(scalings, dtype=scal_dtype).float().numpy()
    n = build_plan(indptr, seg_slots, slot_ranks, scal_f32, n_slots, rows, words)
    meta.plan = torch.from_numpy(words).to(meta.seg_indptr.device)
    meta.plan_cap = cap
    meta.plan_entries = n


def _normal(g: torch.Generator, shape, std: float, mean: float = 0.0) -> torch.Tensor:
    return torch.randn(*shape, generator=g, dtype=torch.float32) * std + mean


def _stacks(g, n_slots, ranks, r_max, in_dim, out_dims, a_std, b_std):
    """A stacks per slice then B stacks per slice; only the first `rank` rows/cols of occupied slots are drawn."""
    a_stacks, b_stacks = [], []
    for _ in out_dims:
        a = torch.zeros(n_slots, r_max, in_dim)
        for slot, r in enumerate(ranks):
            if r > 0:
                a[slot, :r] = _normal(g, (r, in_dim), a_std)
        a_stacks.append(a)
    for out in out_dims:
        b = torch.zeros(n_slots, out, r_max)
        for slot, r in enumerate(ranks):
            if r > 0:
                b[slot, :, :r] = _normal(g, (out, r), b_std)
        b_stacks.append(b)
    return a_stacks, b_stacks


def _finish(name, g, seg_lens, seg_slots, ranks, scalings, x, a_stacks, b_stacks, out_total, dtype, device,
            col_offsets, extra=None, base_std=1.0) -> LoRAWorkload:
    base = _normal(g, (x.shape[0], out_total), base_std)
    dev = torch.device(device)
    cast = lambda t: t.to(dtype).to(dev)  # noqa: E731
    return LoRAWorkload(
        name=name,
        x=cast(x),
        a_stacks=[cast(a) for a in a_stacks],
        b_stacks=[cast(b) for b in b_stacks],
        base=cast(base),
        meta=make_meta(seg_lens, seg_slots, ranks, scalings, dev, dtype),
        col_offsets=col_offsets,
        seg_lens=seg_lens,
        seg_slots=seg_slots,
        slot_ranks=ranks,
        scalings=scalings,
        extra=extra or {},
    )


def cpu_small(device="cpu", dtype=torch.float32) -> LoRAWorkload:
    g = torch.Generator("cpu").manual_seed(0)
    seg_slots, seg_lens = [2, 0, 3], [5, 17, 42]
    ranks, in_dim, out = [8, 8, 8, 8], 1024, 1024
    x = _normal(g, (sum(seg_lens), in_dim), 1.0)
    a, b = _stacks(g, 4, ranks, 8, in_dim, [out], in_dim ** -0.5, 0.02)
    return _finish("cpu_small", g, seg_lens, seg_slots, ranks, [2.0] * 4, x, a, b, out, dtype, device, [0])


def decode_q(device="cpu", dtype=torch.bfloat16, tokens: int = 128, in_dim: int = 4096, out: int = 4096,
             n_slots: int = 64, n_adapters: int = 32, rank: int = 16, seed: int = 1,
             resident: Optional[int] = None) -> LoRAWorkload:
    """Decode tokens, one segment each, over ``n_adapters`` adapters of a pool of ``n_slots``.

    By default the adapters occupy slots 0..n_adapters-1 and the other slots
    are empty (rank 0).  With ``resident`` > n_adapters, slots
    0..resident-1 all hold adapters (as a pool in steady state does) and the
    tokens use a random ``n_adapters`` of them.
    """
    g = torch.Generator("cpu").manual_seed(seed)
    seg_slots = torch.randint(0, n_adapters, (tokens,), generator=g).tolist()
    resident = n_adapters if resident is None else resident
    name = "decode_q"
    if resident > n_adapters:
        used = torch.randperm(resident, generator=g)[:n_adapters].tolist()
        seg_slots = [used[s] for s in seg_slots]
        name = "decode_q_resident"
    seg_lens = [1] * tokens
    ranks = [rank] * resident + [0] * (n_slots - resident)
    x = _normal(g, (tokens, in_dim), 1.0)
    a, b = _stacks(g, n_slots, ranks, rank, in_dim, [out], in_dim ** -0.5, 0.02)
    return _finish(name, g, seg_lens, seg_slots, ranks, [2.0] * n_slots, x, a, b, out, dtype, device, [0])


def prefill_mlp(device="cpu", dtype=torch.bfloat16, part: str = "gate_up", n_seg: int = 8, min_len: int = 64,
                max_len: int = 1024, hidden: int = 4096, inter: int = 14336, r_max: int = 64,
                seed: int = 2) -> LoRAWorkload:
    """``part='gate_up'``: x [S, hidden] -> two slices of width ``inter``; ``part='down'``: [S, inter] -> hidden."""
    g = torch.Generator("cpu").manual_seed(seed)
    seg_slots = list(range(n_seg))
    seg_lens = torch.randint(min_len, max_len + 1, (n_seg,), generator=g).tolist()
    choices = [r for r in (16, 32, 64) if r <= r_max] or [r_max]
    ranks = [choices[i] for i in torch.randint(0, len(choices), (n_seg,), generator=g).tolist()]
    if part == "gate_up":
        in_dim, outs = hidden, [inter, inter]
    else:
        in_dim, outs = inter, [hidden]
    x = _normal(g, (sum(seg_lens), in_dim), 1.0)
    a, b = _stacks(g, n_seg, ranks, r_max, in_dim, outs, in_dim ** -0.5, 0.02)
    cols = [0, inter] if part == "gate_up" else [0]
    return _finish(f"prefill_{part}", g, seg_lens, seg_slots, ranks, [2.0] * n_seg, x, a, b, sum(outs), dtype,
                   device, cols)


def decode_qkv(device="cpu", dtype=torch.bfloat16, tokens: int = 256, hidden: int = 4096,
               outs: Optional[List[int]] = None, n_slots: int = 256, n_adapters: int = 128, rank: int = 32,
               seed: int = 3) -> LoRAWorkload:
    outs = outs or [4096, 1024, 1024]
    g = torch.Generator("cpu").manual_seed(seed)
    seg_slots = torch.randint(0, n_adapters, (tokens,), generator=g).tolist()
    seg_lens = [1] * tokens
    ranks = [rank] * n_adapters + [0] * (n_slots - n_adapters)
    x = _normal(g, (tokens, hidden), 1.0)
    norm_w = _normal(g, (hidden,), 0.1, mean=1.0)
    a, b = _stacks(g, n_slots, ranks, rank, hidden, outs, hidden ** -0.5, 0.02)
    cols, c = [], 0
    for o in outs:
        cols.append(c)
        c += o
    wl = _finish("decode_qkv", g, seg_lens, seg_slots, ranks, [2.0] * n_slots, x, a, b, sum(outs),
                 dtype, device, cols)
    wl.extra["norm_weight"] = norm_w.to(dtype).to(torch.device(device))
    wl.extra["eps"] = 1e-5
    return wl


def mixed_c5(device="cpu", dtype=torch.bfloat16, part: str = "gate_up", hidden: int = 4096, inter: int = 14336,
             kv: int = 1024, n_slots: int = 128, n_adapters: int = 35, rank: int = 16, seed: int = 4) -> LoRAWorkload:
    """One LoRA call of the 32-layer step's mixed batch: 2 prompts of 512 tokens, then 64 decode rows, one
    segment each; a 128-slot pool holding ``n_adapters`` rank-16 adapters, slot per segment uniform over
    them.  ``part`` is ``gate_up`` (4096 -> 2 x 14336), ``qkv`` (4096 -> [4096, 1024, 1024]), ``o``
    (4096 -> 4096) or ``down`` (14336 -> 4096)."""
    g = torch.Generator("cpu").manual_seed(seed)
    seg_lens = [512, 512] + [1] * 64
    seg_slots = torch.randint(0, n_adapters, (len(seg_lens),), generator=g).tolist()
    ranks = [rank] * n_adapters + [0] * (n_slots - n_adapters)
    in_dim, outs = {"gate_up": (hidden, [inter, inter]), "qkv": (hidden, [hidden, kv, kv]), "o": (hidden, [hidden]),
                    "down": (inter, [hidden])}[part]
    x = _normal(g, (sum(seg_lens), in_dim), 1.0)
    a, b = _stacks(g, n_slots, ranks, rank, in_dim, outs, in_dim ** -0.5, 0.02)
    cols, c = [], 0
    for o in outs:
        cols.append(c)
        c += o
    return _finish(f"c5_{part}", g, seg_lens, seg_slots, ranks, [2.0] * n_slots, x, a, b, sum(outs), dtype, device,
                   cols)


def algorithmic_bytes(wl: LoRAWorkload, include_x: bool = True) -> int:
    """HBM bytes a perfect shrink+expand moves: x once, each referenced slot's live A rows and
    B columns once per slice, and the residual read plus write."""
    e = wl.x.element_size()
    used = sorted({s for s, n in zip(wl.seg_slots, wl.seg_lens) if n > 0 and wl.slot_ranks[s] > 0})
    in_dim = wl.x.shape[1]
    total = wl.x.numel() * e if include_x else 0
    for slot in used:
        r = wl.slot_ranks[slot]
        for b in wl.b_stacks:
            total += r * in_dim * e + b.shape[1] * r * e
    out_cols = sum(b.shape[1] for b in wl.b_stacks)
    total += 2 * wl.tokens * out_cols * e
    return total


def flops(wl: LoRAWorkload) -> int:
    in_dim = wl.x.shape[1]
    total = 0
    for s, n in zip(wl.seg_slots, wl.seg_lens):
        r = wl.slot_ranks[s]
        for b in wl.b_stacks:
            total += 2 * n * r * (in_dim + b.shape[1])
    return total
