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


class ReadyTimeCounters:
    """Ready-before-demand accounting on virtual time, restated.

    Reference: src/mtp_expert_prefetch/runtime/cache_manager.py:298-578
    (ReadyTimeExpertCacheManager). Prefetch issues queue up (deduplicated against resident and
    in-flight keys) and are served in batches of `batch` issues by one server: a batch starts
    at max(server free, ready time) and takes per_batch + per_issue * size microseconds; a
    partial batch is released when a request arrives `deadline` microseconds after its first
    issue (never when deadline is 0), or at finish(). A transfer's key enters the LRU as an
    unused prefetch once virtual time reaches its completion; a demand sees the transfers
    completed by arrival + deadline. A demand of a key still in flight is a miss and a
    ready-late miss, and the key is inserted as used; when that transfer later completes, the
    key is already resident (not as a prefetch), which counts as a late completion left unused.
    """

    def __init__(self, capacity: int, per_issue: float = 0.0, per_batch: float = 0.0,
                 batch: int = 1, deadline: float = 0.0) -> None:
        import math
        for name, v in (("per_issue", per_issue), ("per_batch", per_batch),
                        ("deadline", deadline)):
            if not math.isfinite(float(v)):
                raise ValueError(f"{name} must be finite")
        self.lru = LruCounters(capacity)
        self.per_issue = max(0.0, float(per_issue))
        self.per_batch = max(0.0, float(per_batch))
        self.batch = max(1, int(batch) or 1)
        self.deadline = max(0.0, float(deadline))
        self.pending: list[tuple[int, int]] = []
        self.pending_t0: float | None = None  # arrival of the first pending issue
        self.done: list[tuple[float, list[tuple[int, int]]]] = []  # completion order (FIFO)
        self.inflight: set[tuple[int, int]] = set()
        self.server_free = 0.0
        self.last_completion = 0.0
        self.last_arrival = 0.0
        self.ready_late = 0
        self.late_unused = 0
        self.batches = 0
        self.service = 0.0
        self.wait = 0.0
        self.max_delay = 0.0

    # --- the queue
    def _serve(self, keys, ready: float, first: float) -> None:
        if not keys:
            return
        svc = self.per_batch + self.per_issue * len(keys)
        start = max(self.server_free, ready)
        end = start + svc
        self.batches += 1
        self.service += svc
        self.wait += max(0.0, start - ready)
        self.max_delay = max(self.max_delay, end - first)
        self.server_free = end
        self.last_completion = end
        self.done.append((end, list(keys)))

    def _release_full(self, now: float) -> None:
        while len(self.pending) >= self.batch:
            first = now if self.pending_t0 is None else self.pending_t0
            head, self.pending = self.pending[:self.batch], self.pending[self.batch:]
            self._serve(head, now, first)
            self.pending_t0 = now if self.pending else None

    def _release_due(self, now: float) -> None:
        if (self.pending and self.pending_t0 is not None and self.deadline > 0.0
                and now >= self.pending_t0 + self.deadline):
            first = self.pending_t0
            keys, self.pending, self.pending_t0 = self.pending, [], None
            self._serve(keys, first + self.deadline, first)

    def _complete(self, now: float) -> None:
        while self.done and self.done[0][0] <= now:
            _, keys = self.done.pop(0)
            for key in keys:
                self.inflight.discard(key)
                entry = self.lru.cache.get(key)
                if entry is not None:
                    if not entry[0]:
                        self.late_unused += 1
                    self.lru.cache.move_to_end(key)
                else:
                    self.lru._insert(key, True, False)

    # --- the interface
    def advance_to(self, t: float) -> None:
        t = max(0.0, float(t))
        self.last_arrival = max(self.last_arrival, t)
        self._release_due(t)
        self._complete(t)

    def issue_prefetch(self, layer: int, expert: int, t: float) -> bool:
        key = (int(layer), int(expert))
        self.advance_to(t)
        if key in self.lru.cache:
            self.lru.cache.move_to_end(key)
            return False
        if key in self.inflight:
            return False
        self.lru.issued += 1
        self.inflight.add(key)
        if not self.pending:
            self.pending_t0 = float(t)
        self.pending.append(key)
        self._release_full(float(t))
        return True

    def demand(self, layer: int, expert: int, t: float) -> bool:
        due = float(t) + self.deadline
        self._release_due(due)
        self._complete(due)
        key = (int(layer), int(expert))
        if key in self.lru.cache:
            return self.lru.demand(layer, expert)
        if key in self.inflight:
            self.ready_late += 1
        return self.lru.demand(layer, expert)

    def finish(self) -> None:
        if self.pending and self.pending_t0 is not None:
            first = self.pending_t0
            ready = first + self.deadline if self.deadline > 0.0 else self.last_arrival
            keys, self.pending, self.pending_t0 = self.pending, [], None
            self._serve(keys, ready, first)
        self._complete(float("inf"))

    def stats(self) -> dict:
        lru = self.lru
        return {
            "capacity": lru.capacity, "resident_count": len(lru.cache),
            "issued_fetch_count": lru.issued, "used_fetch_count": lru.used,
            "unused_fetch_count": lru.unused() + self.late_unused,
            "demand_count": lru.demand_count, "demand_hit_count": lru.hits,
            "demand_miss_count": lru.misses, "evicted_before_use_count": lru.evicted_before_use,
            "ready_late_miss_count": self.ready_late, "late_completion_unused_count": self.late_unused,
            "queue_batch_count": self.batches, "queue_service_us": self.service,
            "queue_total_span_us": self.last_completion if lru.issued else 0.0,
            "queue_wait_us": self.wait, "queue_max_delay_us": self.max_delay,
            "queue_event_interval_us": 0.0, "queue_deadline_us": self.deadline,
            "queue_batch_size": self.batch,
        }
