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


# ---- ReadyTimeCounters (cache_manager.py:298-578), pinned by the reference's scenarios
# (tests/test_cache_manager.py:64-160) and by its reduction to the plain LRU.
from oracle.cache_ref import ReadyTimeCounters  # noqa: E402


def test_ready_time_hit_only_when_ready_before_the_deadline():
    m = ReadyTimeCounters(2, per_issue=2.0, batch=1, deadline=5.0)
    assert m.issue_prefetch(0, 1, 0.0) is True
    assert m.demand(0, 1, 0.0) is True  # ready at 2 us, deadline 5 us
    s = m.stats()
    assert (s["issued_fetch_count"], s["used_fetch_count"], s["demand_hit_count"],
            s["ready_late_miss_count"], s["queue_batch_count"], s["queue_service_us"]) == (1, 1, 1, 0, 1, 2.0)


def test_ready_time_late_inflight_demand_is_a_miss():
    m = ReadyTimeCounters(2, per_issue=10.0, batch=1, deadline=5.0)
    assert m.issue_prefetch(0, 1, 0.0) is True
    assert m.demand(0, 1, 0.0) is False  # ready at 10 us > 5 us
    m.finish()
    s = m.stats()
    assert (s["issued_fetch_count"], s["used_fetch_count"], s["demand_miss_count"],
            s["ready_late_miss_count"], s["late_completion_unused_count"],
            s["unused_fetch_count"]) == (1, 0, 1, 1, 1, 1)


def test_ready_time_dedups_resident_and_inflight_issues():
    m = ReadyTimeCounters(2, per_issue=10.0, batch=1, deadline=5.0)
    assert m.issue_prefetch(0, 1, 0.0) is True
    assert m.issue_prefetch(0, 1, 1.0) is False  # in flight
    m.advance_to(20.0)
    assert m.issue_prefetch(0, 1, 20.0) is False  # resident
    s = m.stats()
    assert (s["issued_fetch_count"], s["resident_count"]) == (1, 1)


def test_ready_time_capacity_zero_drops_ready_prefetches():
    m = ReadyTimeCounters(0, per_issue=1.0, batch=1, deadline=5.0)
    assert m.issue_prefetch(0, 1, 0.0) is True
    m.finish()
    s = m.stats()
    assert (s["resident_count"], s["issued_fetch_count"], s["evicted_before_use_count"]) == (0, 1, 1)


def test_ready_time_underfilled_batch_released_at_the_deadline():
    m = ReadyTimeCounters(2, per_issue=1.0, batch=2, deadline=5.0)
    assert m.issue_prefetch(0, 1, 0.0) is True
    assert m.demand(0, 1, 0.0) is False  # released at 5 us, ready at 6 us
    m.finish()
    s = m.stats()
    assert (s["queue_batch_count"], s["queue_service_us"], s["queue_total_span_us"],
            s["demand_miss_count"], s["ready_late_miss_count"],
            s["late_completion_unused_count"]) == (1, 1.0, 6.0, 1, 1, 1)


def test_ready_time_invalid_parameters_are_refused():
    import math
    import pytest
    for kw in ({"per_issue": math.inf}, {"per_batch": math.nan}, {"deadline": -math.inf}):
        with pytest.raises(ValueError):
            ReadyTimeCounters(2, **kw)
    m = ReadyTimeCounters(2, per_issue=-3.0, batch=0, deadline=-1.0)  # clamped
    assert (m.per_issue, m.batch, m.deadline) == (0.0, 1, 0.0)


def test_ready_time_batching_and_server_queueing_closed_form():
    """Four issues at t = 0 in batches of 2, per batch 3 us + 1 us per issue: the batches take
    5 us each and the second waits for the first (start 5, end 10)."""
    m = ReadyTimeCounters(8, per_issue=1.0, per_batch=3.0, batch=2, deadline=0.0)
    for e in range(4):
        m.issue_prefetch(0, e, 0.0)
    s = m.stats()
    assert (s["queue_batch_count"], s["queue_service_us"], s["queue_wait_us"],
            s["queue_max_delay_us"], s["queue_total_span_us"]) == (2, 10.0, 5.0, 10.0, 10.0)
    assert m.demand(0, 0, 4.9) is False and m.demand(0, 1, 5.0) is True  # first batch at 5 us
    assert m.demand(0, 2, 9.9) is False and m.ready_late == 2


def test_ready_time_with_zero_service_reduces_to_the_lru():
    """With no service time and no deadline every issue is ready at its own arrival, so on
    nondecreasing arrivals the counters equal those of the plain LRU (ControlledExpertCacheManager)
    for any sequence; a planted off-by-one in the completion rule (strict < instead of <=) makes
    every prefetch late and must fail."""
    import random
    rng = random.Random(3)
    for trial in range(50):
        cap = rng.randint(0, 6)
        lru, rt = LruCounters(cap), ReadyTimeCounters(cap)
        t = 0.0
        for _ in range(200):
            t += rng.choice((0.0, 0.5, 1.0))
            layer, e = rng.randrange(2), rng.randrange(10)
            if rng.random() < 0.5:
                assert lru.issue_prefetch(layer, e) == rt.issue_prefetch(layer, e, t)
            else:
                rt.advance_to(t)
                assert lru.demand(layer, e) == rt.demand(layer, e, t)
        rt.finish()  # the last issue completes at its own arrival
        s = rt.stats()
        assert (s["issued_fetch_count"], s["used_fetch_count"], s["demand_hit_count"],
                s["demand_miss_count"], s["evicted_before_use_count"], s["resident_count"],
                s["ready_late_miss_count"]) == (lru.issued, lru.used, lru.hits, lru.misses,
                                                lru.evicted_before_use, len(lru.cache), 0)

    class Strict(ReadyTimeCounters):
        def _complete(self, now):
            while self.done and self.done[0][0] < now:
                _, keys = self.done.pop(0)
                for key in keys:
                    self.inflight.discard(key)
                    if key not in self.lru.cache:
                        self.lru._insert(key, True, False)
    bad = Strict(4)
    bad.issue_prefetch(0, 1, 0.0)
    assert bad.demand(0, 1, 0.0) is False  # the planted mistake is caught
