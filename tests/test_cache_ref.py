"""Pins the slot-cache counter oracle against the reference's scenarios
(tests/test_cache_manager.py:21-62, ControlledExpertCacheManager)."""

from __future__ import annotations

from oracle.cache_ref import LruCounters


def test_tracks_prefetch_use_and_miss():
    m = LruCounters(2)
    assert m.issue_prefetch(0, 1) is True
    assert m.issue_prefetch(0, 1) is False
    assert m.demand(0, 1) is True
    assert m.demand(0, 2) is False
    assert (m.issued, m.used, m.demand_count, m.hits, m.misses, m.unused()) == (1, 1, 2, 1, 1, 0)


def test_counts_evicted_unused_prefetches():
    m = LruCounters(1)
    m.issue_prefetch(0, 1)
    m.issue_prefetch(0, 2)
    m.demand(0, 1)
    assert (m.issued, m.evicted_before_use, m.misses, m.used) == (2, 2, 1, 0)


def test_capacity_zero_drops_prefetches():
    m = LruCounters(0)
    m.issue_prefetch(0, 1)
    m.demand(0, 1)
    assert (len(m.cache), m.issued, m.evicted_before_use, m.misses) == (0, 1, 1, 1)
