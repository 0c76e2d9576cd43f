"""LRU expert slot-cache counter semantics, restated.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference: src/mtp_expert_prefetch/runtime/cache_manager.py:208-279
(ControlledExpertCacheManager). Keys are (layer, expert); capacity is the number
of resident entries; a prefetch of a resident key only refreshes its recency; a
demand miss inserts the key as used; evicting (or dropping at capacity 0) a
prefetched-but-unused entry counts as evicted-before-use.
"""

from __future__ import annotations

from collections import OrderedDict


class LruCounters:
    def __init__(self, capacity: int) -> None:
        self.capacity = int(capacity)
        self.cache: OrderedDict[tuple[int, int], list[bool]] = OrderedDict()  # key -> [prefetched, used]
        self.issued = 0
        self.used = 0
        self.demand_count = 0
        self.hits = 0
        self.misses = 0
        self.evicted_before_use = 0

    def _insert(self, key, prefetched: bool, used: bool) -> None:
        if self.capacity <= 0:
            if prefetched and not used:
                self.evicted_before_use += 1
            return
        self.cache[key] = [prefetched, used]
        self.cache.move_to_end(key)
        while len(self.cache) > self.capacity:
            _, (p, u) = self.cache.popitem(last=False)
            if p and not u:
                self.evicted_before_use += 1

    def issue_prefetch(self, layer: int, expert: int) -> bool:
        key = (int(layer), int(expert))
        if key in self.cache:
            self.cache.move_to_end(key)
            return False
        self.issued += 1
        self._insert(key, True, False)
        return True

    def demand(self, layer: int, expert: int) -> bool:
        self.demand_count += 1
        key = (int(layer), int(expert))
        entry = self.cache.get(key)
        if entry is None:
            self.misses += 1
            self._insert(key, False, True)
            return False
        self.hits += 1
        if entry[0] and not entry[1]:
            self.used += 1
        entry[1] = True
        self.cache.move_to_end(key)
        return True

    def unused(self) -> int:
        return sum(1 for p, u in self.cache.values() if p and not u)
