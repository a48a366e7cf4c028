"""CPU restatement of slot allocation and eviction (test infrastructure).

Follows multi_lora/pool.py:382-420,443-473 and multi_lora/eviction.py:12-50:
mark every adapter of the batch as used, then for each non-resident one take
the lowest empty slot, or else evict — among resident adapters not in the
batch — the one first in the policy's order; the base model (``None``) is
never queued and is evicted only when nothing else can be.
"""

from __future__ import annotations

from typing import Dict, List, Optional


class SlotPoolRef:
    def __init__(self, num_slots: int, kind: str = "lru") -> None:
        assert kind in ("lru", "fifo")
        self.num_slots = num_slots
        self.kind = kind
        self.order: List[str] = []  # front = evicted first
        self.slot_of: Dict[Optional[str], int] = {}
        self.evictions = 0

    def _use(self, name: Optional[str]) -> None:
        if name is None:
            return
        if name in self.order:
            if self.kind == "lru":
                self.order.remove(name)
                self.order.append(name)
        else:
            self.order.append(name)

    def prepare(self, names: List[Optional[str]]) -> List[Optional[str]]:
        """Make ``names`` resident; returns the adapters that had to be loaded."""
        batch = list(dict.fromkeys(names))
        for n in batch:
            self._use(n)
        loaded = []
        for n in batch:
            if n in self.slot_of:
                continue
            used = set(self.slot_of.values())
            free = [s for s in range(self.num_slots) if s not in used]
            if free:
                slot = free[0]
            else:
                victims = [v for v in self.order if v in self.slot_of and v not in batch]
                if victims:
                    victim = victims[0]
                elif None in self.slot_of and None not in batch:
                    victim = None
                else:
                    raise ValueError("no evictable slot")
                slot = self.slot_of.pop(victim)
                if victim is not None:
                    self.order.remove(victim)
                self.evictions += 1
            self.slot_of[n] = slot
            loaded.append(n)
        return loaded
