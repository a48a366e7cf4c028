"""Victim selection for a full slot pool: LRU or FIFO.

Same policy as multi_lora/eviction.py:12-50:
* ``lru``  — every use moves the adapter to the back; the front is evicted.
* ``fifo`` — an adapter is queued on first use only.
The base model (``None``) is never queued; it is chosen only when no queued
candidate remains.
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Iterable, Optional

POLICIES = ("lru", "fifo")


class EvictionPolicy:
    def __init__(self, kind: str = "lru") -> None:
        if kind not in POLICIES:
            raise ValueError(f"unknown eviction policy: {kind}; try lru | fifo")
        self.kind = kind
        self.order: "OrderedDict[str, None]" = OrderedDict()
        self.eviction_count = 0

    def mark_used(self, name: Optional[str]) -> None:
        if name is None:
            return
        if self.kind == "lru" and name in self.order:
            self.order.move_to_end(name)
        elif name not in self.order:
            self.order[name] = None

    def select_victim(self, candidates: Iterable[Optional[str]]) -> Optional[str]:
        pool = set(candidates)
        victim = next((name for name in self.order if name in pool), _NO_VICTIM)
        if victim is _NO_VICTIM:
            if None not in pool:
                raise RuntimeError(f"no evictable adapter in {pool}")
            victim = None
        self.eviction_count += 1
        return victim

    def remove(self, name: Optional[str]) -> None:
        if name is not None:
            self.order.pop(name, None)


_NO_VICTIM = object()
