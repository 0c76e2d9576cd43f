"""The reference's cache-lab expert-payload managers on the library's native accounting.

Same names, constructor arguments, methods and snapshot fields as
src/mtp_expert_prefetch/runtime/cache_manager.py:
  * ControlledExpertCacheManager (:208-279): one LRU of `capacity` (layer, expert) keys; a
    prefetch of a missing key enters it at once.
  * ReadyTimeExpertCacheManager (:298-578): prefetches are transfers served by one virtual queue
    (service time per issue and per batch, batching, a release deadline); a demand hits only
    keys whose transfer completed by its arrival + queue_deadline_us, and a demand of a key
    still in flight is a ready-late miss.

Both run in libmoe_w4a16.so (moe_ready_cache_*_v1, host code, no HIP call). The slot cache that
moves the bytes (mtp_amd.offload.SlotCache) keeps its own per-layer LRU and measures readiness
with HIP events; feeding the same call sequence, with arrival times, to a
ReadyTimeExpertCacheManager gives the reference-semantics counters beside it.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import asdict, dataclass

from mtp_amd import _lib

_CONTROLLED, _READY_TIME = 0, 1


@dataclass(frozen=True)
class CacheManagerSnapshot:
    capacity: int
    resident_count: int
    issued_fetch_count: int
    used_fetch_count: int
    unused_fetch_count: int
    demand_count: int
    demand_hit_count: int
    demand_miss_count: int
    evicted_before_use_count: int

    def as_dict(self) -> dict:
        return asdict(self)


@dataclass(frozen=True)
class ReadyTimeCacheManagerSnapshot(CacheManagerSnapshot):
    ready_late_miss_count: int
    late_completion_unused_count: int
    queue_batch_count: int
    queue_service_us: float
    queue_total_span_us: float
    queue_wait_us: float
    queue_max_delay_us: float
    queue_event_interval_us: float
    queue_deadline_us: float
    queue_batch_size: int


class _NativeManager:
    def __init__(self, mode: int, capacity: int, per_issue: float, per_batch: float,
                 batch: int, deadline: float) -> None:
        self._lib = _lib.load()
        self._handle = ctypes.c_uint64(0)
        _lib.check(self._lib.moe_ready_cache_create_v1(mode, int(capacity), per_issue, per_batch,
                                                       int(batch), deadline,
                                                       ctypes.byref(self._handle)))
        self.capacity = int(capacity)

    def __del__(self) -> None:
        h = getattr(self, "_handle", None)
        if h is not None and h.value:
            self._lib.moe_ready_cache_destroy_v1(h)
            h.value = 0

    def _call(self, fn, layer: int, experts, arrival_us: float) -> list[bool]:
        ids = [int(e) for e in experts]
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        flags = (ctypes.c_int32 * max(1, len(ids)))()
        count = ctypes.c_int32()
        _lib.check(fn(self._handle, int(layer), arr, len(ids), float(arrival_us), flags,
                      ctypes.byref(count)))
        return [bool(flags[i]) for i in range(len(ids))]

    def _stats(self) -> _lib.ReadyCacheStats:
        st = _lib.ReadyCacheStats()
        _lib.check(self._lib.moe_ready_cache_stats_v1(self._handle, ctypes.byref(st)))
        return st


class ControlledExpertCacheManager(_NativeManager):
    """Bounded LRU expert-payload cache (cache_manager.py:208-279)."""

    def __init__(self, *, capacity: int) -> None:
        super().__init__(_CONTROLLED, capacity, 0.0, 0.0, 1, 0.0)

    def issue_prefetch(self, layer_idx: int, expert_idx: int) -> bool:
        return self._call(self._lib.moe_ready_cache_prefetch_v1, layer_idx, [expert_idx], 0.0)[0]

    def demand(self, layer_idx: int, expert_idx: int) -> bool:
        return self._call(self._lib.moe_ready_cache_demand_v1, layer_idx, [expert_idx], 0.0)[0]

    def snapshot(self) -> CacheManagerSnapshot:
        st = self._stats()
        return CacheManagerSnapshot(**{f: int(getattr(st, f))
                                       for f in CacheManagerSnapshot.__dataclass_fields__})


class ReadyTimeExpertCacheManager(_NativeManager):
    """Bounded expert-payload cache with ready-before-demand semantics on virtual time
    (cache_manager.py:298-578)."""

    def __init__(self, *, capacity: int, service_us_per_issue: float = 0.0,
                 service_us_per_batch: float = 0.0, queue_batch_size: int = 1,
                 queue_deadline_us: float = 0.0) -> None:
        per_issue, per_batch, deadline = (float(service_us_per_issue),
                                          float(service_us_per_batch), float(queue_deadline_us))
        for name, value in (("service_us_per_issue", per_issue),
                            ("service_us_per_batch", per_batch),
                            ("queue_deadline_us", deadline)):
            if not math.isfinite(value):
                raise ValueError(f"{name} must be finite")
        super().__init__(_READY_TIME, capacity, per_issue, per_batch,
                         max(1, int(queue_batch_size) or 1), deadline)
        self.service_us_per_issue = max(0.0, per_issue)
        self.service_us_per_batch = max(0.0, per_batch)
        self.queue_batch_size = max(1, int(queue_batch_size) or 1)
        self.queue_deadline_us = max(0.0, deadline)

    def issue_prefetch(self, layer_idx: int, expert_idx: int, *, arrival_us: float) -> bool:
        return self._call(self._lib.moe_ready_cache_prefetch_v1, layer_idx, [expert_idx],
                          arrival_us)[0]

    def issue_prefetches(self, layer_idx: int, expert_indices, *, arrival_us: float) -> int:
        return sum(self._call(self._lib.moe_ready_cache_prefetch_v1, layer_idx,
                              list(expert_indices), arrival_us))

    def demand(self, layer_idx: int, expert_idx: int, *, arrival_us: float) -> bool:
        return self._call(self._lib.moe_ready_cache_demand_v1, layer_idx, [expert_idx],
                          arrival_us)[0]

    def demand_many(self, layer_idx: int, expert_indices, *, arrival_us: float) -> list[bool]:
        """demand() of each expert in order at one arrival time (one native call)."""
        return self._call(self._lib.moe_ready_cache_demand_v1, layer_idx, list(expert_indices),
                          arrival_us)

    def advance_to(self, arrival_us: float) -> None:
        _lib.check(self._lib.moe_ready_cache_advance_v1(self._handle, float(arrival_us)))

    def finish(self) -> None:
        _lib.check(self._lib.moe_ready_cache_finish_v1(self._handle))

    def snapshot(self) -> ReadyTimeCacheManagerSnapshot:
        st = self._stats()
        vals = {}
        for f, t in ReadyTimeCacheManagerSnapshot.__dataclass_fields__.items():
            v = getattr(st, f)
            vals[f] = float(v) if t.type in ("float", float) else int(v)
        return ReadyTimeCacheManagerSnapshot(**vals)
