"""Adapter slot pool: K device slots per LoRA module, filled on demand.

Mirrors the reference's ``LoRAMemoryPool`` (multi_lora/pool.py:325-473) and
its slot tensors (pool.py:97-155):

* per module key, ``A[key]`` is ``[K, max_lora_rank, in]`` and ``B[key]`` is
  ``[K, out, max_lora_rank]`` in the model dtype, zero-initialised; the
  kernels read only the first ``rank`` rows of A / columns of B of a slot;
* ``name_to_slot`` / ``slot_names`` / ``_slot_rank_scaling`` map adapters to
  slots; ``None`` is the base model (rank 0, scaling 0, no weights);
* a full pool evicts an adapter that is not in the current batch, chosen by
  the eviction policy; the base slot goes last (pool.py:443-473).

Upload.  The first time an adapter is loaded its weights are packed once
into a flat host bank (pinned when the pool is on a GPU), kept on the
adapter object: all A blocks, then all B blocks, at offsets fixed per rank
(the same packing the reference uses, pool.py:23-58).  A reload is then one contiguous H2D copy of the bank into a
device staging row, on a side stream ordered after the compute stream; one
``mlora_pool_scatter`` launch per staged chunk then copies every key's
blocks into the slots (the reference's scatter kernel,
multi_lora/kernels/scatter_bank.py:17-93).  The compute stream waits for the
upload before the next forward.  A pool on the CPU (host logic and tests)
copies with torch instead.
"""

from __future__ import annotations

from typing import Dict, Iterable, List, Optional, Tuple

import ctypes

import torch

from . import _ffi
from .batch_info import BatchLoRAInfo
from .eviction import EvictionPolicy
from .weights import AdapterWeights

LoraName = Optional[str]

# Adapters staged per device round trip; bounds the staging buffer.
_BANK_CHUNK = 4


class _RankPlan:
    """Flat bank layout for one rank: every key's A block, then every B block."""

    def __init__(self, rank: int, keys: List[str], dims: Dict[str, Tuple[int, int]]):
        self.rank = rank
        self.keys = keys
        self.a_off: Dict[str, int] = {}
        self.b_off: Dict[str, int] = {}
        self.a_shape: Dict[str, Tuple[int, int]] = {}
        self.b_shape: Dict[str, Tuple[int, int]] = {}
        cursor = 0
        for key in keys:
            in_dim = dims[key][0]
            self.a_off[key], self.a_shape[key] = cursor, (rank, in_dim)
            cursor += rank * in_dim
        for key in keys:
            out_dim = dims[key][1]
            self.b_off[key], self.b_shape[key] = cursor, (out_dim, rank)
            cursor += out_dim * rank
        self.total = cursor
        self.dims = dims
        self.device_table: Optional[torch.Tensor] = None  # mlora_pool_key[len(keys)] on the device
        self.max_numel = max([rank * dims[k][0] for k in keys] + [dims[k][1] * rank for k in keys] + [0])
        self.tables: Optional[dict] = None

    def build_tables(self, buffers: "_GpuBuffers", device) -> dict:
        """The scatter tables of this layout over ``buffers``' slot tensors, built
        once (the slot tensors keep their addresses while the key set holds):
        ``keys`` (the mlora_pool_key array on the device), ``n`` keys,
        ``max_numel`` and ``num_slots``; what ``kernels.scatter_stage`` takes,
        as the reference's ``_RankPlan.build_tables`` feeds its scatter kernel
        (multi_lora/pool.py:60-96)."""
        if self.tables is None:
            arr = (_ffi.PoolKey * len(self.keys))()
            for j, key in enumerate(self.keys):
                a, b = buffers.A[key], buffers.B[key]
                arr[j] = _ffi.PoolKey(a.data_ptr(), a.stride(0), self.a_off[key], b.data_ptr(), b.stride(0),
                                      b.stride(1), self.b_off[key], a.shape[2], b.shape[1])
            host = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8)
            self.device_table = host.to(device)
            self.tables = {"keys": self.device_table, "n": len(self.keys), "max_numel": self.max_numel,
                           "num_slots": buffers.max_loras_per_batch}
        return self.tables


class _GpuBuffers:
    """The slot tensors of every module key, plus the upload machinery."""

    def __init__(self, max_loras_per_batch: int, max_lora_rank: int, device: torch.device, dtype: torch.dtype):
        self.max_loras_per_batch = max_loras_per_batch
        self.max_lora_rank = max_lora_rank
        self.device = torch.device(device)
        self.dtype = dtype
        self.A: Dict[str, torch.Tensor] = {}
        self.B: Dict[str, torch.Tensor] = {}
        # Bank layouts by (module signature, rank); the signature lists every
        # module key with its (in, out) widths and grows with ensure().
        self._layouts: Dict[Tuple[tuple, int], _RankPlan] = {}
        self._signature: tuple = ()
        self._stage: Optional[torch.Tensor] = None
        self._copy_stream = None
        self._load_event = None
        self._last_read: Dict[int, "torch.cuda.Event"] = {}
        # Release the per-module host tensors once an adapter is packed into
        # its bank, so host memory holds one copy of the weights.
        self.release_modules = True

    # -- allocation ---------------------------------------------------------
    def ensure(self, weights: AdapterWeights) -> None:
        """Allocate zeroed slot tensors for module keys seen for the first time."""
        for key, (a, b) in weights.modules.items():
            if key in self.A:
                continue
            in_dim, out_dim = int(a.shape[1]), int(b.shape[0])
            k, r = self.max_loras_per_batch, self.max_lora_rank
            self.A[key] = torch.zeros((k, r, in_dim), device=self.device, dtype=self.dtype)
            self.B[key] = torch.zeros((k, out_dim, r), device=self.device, dtype=self.dtype)
        if len(self._signature) != len(self.A):
            self._signature = tuple((k, int(self.A[k].shape[2]), int(self.B[k].shape[1])) for k in self.A)

    def get(self, key: str) -> Tuple[torch.Tensor, torch.Tensor]:
        if key not in self.A:
            raise KeyError(f"module {key!r} not in pool")
        return self.A[key], self.B[key]

    # -- upload -------------------------------------------------------------
    def write_many(self, pairs: List[Tuple[int, AdapterWeights]]) -> None:
        """Load adapters into their slots: ``pairs = [(slot, weights), ...]``."""
        if not pairs:
            return
        if self.device.type != "cuda":
            self._load(pairs, non_blocking=False)
            return
        if self._copy_stream is None:
            self._copy_stream = torch.cuda.Stream(device=self.device)
            self._load_event = torch.cuda.Event()
        # A slot being overwritten may still be read by queued compute work:
        # wait for the last compute that read it, and nothing else, so an
        # upload overlaps compute on the other slots.
        waited = set()
        for slot, _ in pairs:
            ev = self._last_read.get(slot)
            if ev is not None and id(ev) not in waited:
                self._copy_stream.wait_event(ev)
                waited.add(id(ev))
        with torch.cuda.stream(self._copy_stream):
            self._load(pairs, non_blocking=True)
        self._load_event.record(self._copy_stream)

    def mark_read(self, slots: Iterable[int]) -> None:
        """Record that compute enqueued so far on the current stream reads ``slots``."""
        slots = list(slots)
        if self.device.type != "cuda" or not slots:
            return
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        for slot in slots:
            self._last_read[slot] = ev

    def wait_load(self) -> None:
        """Make the compute stream wait for the last upload."""
        if self._load_event is not None:
            torch.cuda.current_stream(self.device).wait_event(self._load_event)

    def layout(self, rank: int) -> _RankPlan:
        """The upload bank layout of a rank-``rank`` adapter over the pool's current module keys."""
        plan = self._layouts.get((self._signature, rank))
        if plan is None:
            keys = [k for k, _, _ in self._signature]
            plan = _RankPlan(rank, keys, {k: (i, o) for k, i, o in self._signature})
            plan.signature = self._signature
            self._layouts[(self._signature, rank)] = plan
        return plan

    def bank(self, weights: AdapterWeights, plan: _RankPlan) -> torch.Tensor:
        """The adapter's flat upload bank for ``plan``, packed on first use.

        The bank is kept on the adapter object (``weights.banks``), so it
        lives exactly as long as the caller keeps the adapter, and one bank
        serves every pool with the same layout.  With ``release_modules`` the
        per-module tensors are dropped after packing; such an adapter can no
        longer be packed for a different layout (a pool that grew new module
        keys afterwards), which raises rather than upload zeros.
        """
        key = (plan.signature, plan.rank, self.dtype)
        bank = weights.banks.get(key)
        if bank is not None:
            return bank
        if weights.flattened:
            raise RuntimeError(
                f"rank-{plan.rank} adapter's module tensors were released after packing for another module "
                f"layout; the pool now has {len(plan.keys)} module keys and the bank cannot be rebuilt")
        bank = self._pack(weights, plan)
        weights.banks = {key: bank}
        if self.release_modules:
            weights.modules = {}
            weights.flattened = True
        return bank

    def _pack(self, weights: AdapterWeights, plan: _RankPlan) -> torch.Tensor:
        """One host copy in the layout's order: every key's A block, then every
        B block; a module the adapter lacks contributes zeros."""
        pieces = []
        for side in (0, 1):
            for key in plan.keys:
                mod = weights.modules.get(key)
                shape = plan.a_shape[key] if side == 0 else plan.b_shape[key]
                if mod is None:
                    pieces.append(torch.zeros(shape[0] * shape[1], dtype=self.dtype))
                else:
                    pieces.append(mod[side].reshape(-1).to(self.dtype))
        bank = torch.empty(plan.total, dtype=self.dtype, pin_memory=self.device.type == "cuda")
        torch.cat(pieces, out=bank)
        return bank

    def _stage_rows(self, total: int) -> torch.Tensor:
        need = _BANK_CHUNK * total
        if self._stage is None or self._stage.numel() < need:
            self._stage = torch.empty(need, device=self.device, dtype=self.dtype)
        return self._stage[:need].view(_BANK_CHUNK, total)

    def _load(self, pairs: List[Tuple[int, AdapterWeights]], non_blocking: bool) -> None:
        by_rank: Dict[int, List[Tuple[int, AdapterWeights]]] = {}
        for slot, w in pairs:
            by_rank.setdefault(int(w.rank), []).append((slot, w))
        for rank, group in by_rank.items():
            plan = self.layout(rank)
            if self.device.type == "cuda":
                stage = self._stage_rows(plan.total)
                stage.record_stream(torch.cuda.current_stream(self.device))
            for c0 in range(0, len(group), _BANK_CHUNK):
                chunk = group[c0 : c0 + _BANK_CHUNK]
                if self.device.type != "cuda":
                    for slot, w in chunk:
                        self._scatter(self.bank(w, plan), slot, plan)
                    continue
                for i, (slot, w) in enumerate(chunk):
                    stage[i].copy_(self.bank(w, plan), non_blocking=non_blocking)
                self._scatter_staged(stage, [slot for slot, _ in chunk], plan)

    def _key_table(self, plan: _RankPlan) -> torch.Tensor:
        """The plan's mlora_pool_key array on the device, built once per plan."""
        return plan.build_tables(self, self.device)["keys"]

    def _scatter_staged(self, stage: torch.Tensor, slots: List[int], plan: _RankPlan) -> None:
        """One launch: staged rows [0, len(slots)) into their slots, every key."""
        from .kernels.scatter_bank import scatter_stage

        # From pinned memory, so the host does not wait for the copies queued before it.
        slots_dev = torch.tensor(slots, dtype=torch.int32).pin_memory().to(self.device, non_blocking=True)
        scatter_stage(stage, slots_dev, plan.build_tables(self, self.device), plan.total, len(slots), plan.rank)

    def _scatter(self, flat: torch.Tensor, slot: int, plan: _RankPlan) -> None:
        """Copy one adapter's packed blocks into slot ``slot`` (first ``rank`` rows / columns)."""
        r = plan.rank
        for key in plan.keys:
            ao, bo = plan.a_off[key], plan.b_off[key]
            a_shape, b_shape = plan.a_shape[key], plan.b_shape[key]
            self.A[key][slot, :r].copy_(flat[ao : ao + r * a_shape[1]].view(a_shape))
            self.B[key][slot, :, :r].copy_(flat[bo : bo + b_shape[0] * r].view(b_shape))


class LoRAMemoryPool:
    """K device slots; each holds nothing, the base model, or one adapter."""

    def __init__(
        self,
        max_loras_per_batch: int,
        max_lora_rank: int,
        device: torch.device,
        dtype: torch.dtype = torch.float16,
        eviction_policy: str = "lru",
    ) -> None:
        self.max_loras_per_batch = max_loras_per_batch
        self.max_lora_rank = max_lora_rank
        self.device = torch.device(device)
        self.dtype = dtype
        self.eviction_policy = EvictionPolicy(eviction_policy)
        self.name_to_slot: Dict[LoraName, int] = {}
        self.slot_names: Dict[int, LoraName] = {}
        self._slot_rank_scaling: Dict[int, Tuple[int, float]] = {}
        self.buffers = _GpuBuffers(max_loras_per_batch, max_lora_rank, self.device, dtype)
        self._batch_slots: List[int] = []

    def get_slot_id(self, name: LoraName) -> int:
        if name not in self.name_to_slot:
            raise KeyError(f"lora {name!r} not resident in pool")
        return self.name_to_slot[name]

    def get_module_buffers(self, module_key: str) -> Tuple[torch.Tensor, torch.Tensor]:
        return self.buffers.get(module_key)

    def get_slot_weights(self, slot: int, module_key: str) -> Tuple[torch.Tensor, torch.Tensor]:
        a, b = self.buffers.get(module_key)
        return a[slot], b[slot]

    def ensure_buffers(self, weights: AdapterWeights) -> None:
        self.buffers.ensure(weights)

    def prepare_lora_batch(
        self, lora_names: Iterable[LoraName], *, weight_store: Dict[LoraName, AdapterWeights]
    ) -> None:
        """Make every adapter of the batch resident, evicting others as needed.

        Adapters are visited in the iteration order of ``lora_names`` (pass an
        ordered, de-duplicated list for a reproducible slot assignment).  All
        uploads of the batch are issued together on the copy stream, then the
        current (compute) stream is ordered after them.

        Ordering against compute: a batch's slots count as read by all compute
        enqueued on the current stream until the next call; an upload into an
        evicted slot waits for the compute that last read that slot and for
        nothing else.  So the next batch can be prepared while this batch's
        forward is still running, and its uploads overlap that forward
        unless they evict one of its adapters.
        """
        # The previous batch's slots are read by the compute enqueued since it was prepared.
        self.buffers.mark_read(self._batch_slots)
        wanted = list(dict.fromkeys(lora_names))
        keep = set(wanted)
        for name in wanted:
            self.eviction_policy.mark_used(name)
        pairs: List[Tuple[int, AdapterWeights]] = []
        for name in wanted:
            if name in self.name_to_slot:
                continue
            slot = self._alloc_slot(keep)
            self.name_to_slot[name] = slot
            self.slot_names[slot] = name
            if name is None:
                self._slot_rank_scaling[slot] = (0, 0.0)
                continue
            weights = weight_store[name]
            if weights.rank > self.max_lora_rank:
                raise ValueError(f"adapter {name!r} rank {weights.rank} > max_lora_rank {self.max_lora_rank}")
            self.buffers.ensure(weights)
            self._slot_rank_scaling[slot] = (int(weights.rank), float(weights.scaling))
            pairs.append((slot, weights))
        self.buffers.write_many(pairs)
        self.buffers.wait_load()
        self._batch_slots = [self.name_to_slot[n] for n in wanted]

    def build_batch_info(self, lora_names: List[LoraName]) -> BatchLoRAInfo:
        """Slot per segment; rank and scaling per slot (empty slots: 0, 0.0)."""
        k = self.max_loras_per_batch
        ranks = [0] * k
        scalings = [0.0] * k
        for slot, (rank, scaling) in self._slot_rank_scaling.items():
            ranks[slot] = rank
            scalings[slot] = scaling
        return BatchLoRAInfo(
            weight_indices=[self.get_slot_id(n) for n in lora_names],
            lora_ranks=ranks,
            scalings=scalings,
        )

    def _alloc_slot(self, keep_names: set) -> int:
        """An empty slot if any (lowest index), else the slot of an evicted adapter."""
        for slot in range(self.max_loras_per_batch):
            if slot not in self.slot_names:
                return slot
        candidates = {n for n in self.slot_names.values() if n not in keep_names and n is not None}
        if not candidates:
            base_free = any(n is None and n not in keep_names for n in self.slot_names.values())
            if not base_free:
                raise ValueError("no evictable slot: batch needs more adapters than max_loras_per_batch")
            candidates = {None}
        victim = self.eviction_policy.select_victim(candidates)
        slot = self.name_to_slot.pop(victim)
        self.eviction_policy.remove(victim)
        del self.slot_names[slot]
        self._slot_rank_scaling.pop(slot, None)
        return slot

