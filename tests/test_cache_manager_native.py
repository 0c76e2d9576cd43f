"""The reference's cache-lab managers (ControlledExpertCacheManager,
ReadyTimeExpertCacheManager; src/mtp_expert_prefetch/runtime/cache_manager.py:208-578) on the
library's native accounting (moe_ready_cache_*_v1, host code: these tests need no GPU).

* The reference's own scenarios (tests/test_cache_manager.py:21-160), replayed through the same
  method names and snapshot fields.
* Random call sequences against the oracle restatement (oracle/cache_ref.py), counter for
  counter, in both modes and with batching, service times and deadlines.
"""

from __future__ import annotations

import math
import random

import pytest

from mtp_amd import _lib
from mtp_amd.cache_manager import ControlledExpertCacheManager, ReadyTimeExpertCacheManager
from oracle.cache_ref import LruCounters, ReadyTimeCounters


@pytest.fixture(autouse=True)
def _lib_loaded():
    try:
        _lib.load()
    except RuntimeError as exc:
        pytest.skip(str(exc))


def test_controlled_tracks_prefetch_use_and_miss():
    m = ControlledExpertCacheManager(capacity=2)
    assert m.issue_prefetch(0, 1) is True
    assert m.issue_prefetch(0, 1) is False
    assert m.demand(0, 1) is True
    assert m.demand(0, 2) is False
    s = m.snapshot()
    assert (s.issued_fetch_count, s.used_fetch_count, s.demand_count, s.demand_hit_count,
            s.demand_miss_count, s.unused_fetch_count) == (1, 1, 2, 1, 1, 0)


def test_controlled_counts_evicted_unused_prefetches():
    m = ControlledExpertCacheManager(capacity=1)
    m.issue_prefetch(0, 1)
    m.issue_prefetch(0, 2)
    m.demand(0, 1)
    s = m.snapshot()
    assert (s.issued_fetch_count, s.evicted_before_use_count, s.demand_miss_count,
            s.used_fetch_count) == (2, 2, 1, 0)


def test_controlled_capacity_zero_drops_prefetches():
    m = ControlledExpertCacheManager(capacity=0)
    m.issue_prefetch(0, 1)
    m.demand(0, 1)
    s = m.snapshot()
    assert (s.resident_count, s.issued_fetch_count, s.evicted_before_use_count,
            s.demand_miss_count) == (0, 1, 1, 1)


def test_ready_time_hits_only_after_ready_before_deadline():
    m = ReadyTimeExpertCacheManager(capacity=2, service_us_per_issue=2.0, queue_batch_size=1,
                                    queue_deadline_us=5.0)
    assert m.issue_prefetch(0, 1, arrival_us=0.0) is True
    assert m.demand(0, 1, arrival_us=0.0) is True
    s = m.snapshot()
    assert (s.issued_fetch_count, s.used_fetch_count, s.demand_hit_count, s.ready_late_miss_count,
            s.queue_batch_count, s.queue_service_us) == (1, 1, 1, 0, 1, 2.0)


def test_ready_time_counts_late_inflight_miss():
    m = ReadyTimeExpertCacheManager(capacity=2, service_us_per_issue=10.0, queue_batch_size=1,
                                    queue_deadline_us=5.0)
    assert m.issue_prefetch(0, 1, arrival_us=0.0) is True
    assert m.demand(0, 1, arrival_us=0.0) is False
    m.finish()
    s = m.snapshot()
    assert (s.issued_fetch_count, s.used_fetch_count, s.demand_miss_count,
            s.ready_late_miss_count, s.late_completion_unused_count,
            s.unused_fetch_count) == (1, 0, 1, 1, 1, 1)


def test_ready_time_deduplicates_resident_and_inflight_issue():
    m = ReadyTimeExpertCacheManager(capacity=2, service_us_per_issue=10.0, queue_batch_size=1,
                                    queue_deadline_us=5.0)
    assert m.issue_prefetch(0, 1, arrival_us=0.0) is True
    assert m.issue_prefetch(0, 1, arrival_us=1.0) is False
    m.advance_to(20.0)
    assert m.issue_prefetch(0, 1, arrival_us=20.0) is False
    s = m.snapshot()
    assert (s.issued_fetch_count, s.resident_count) == (1, 1)


def test_ready_time_capacity_zero_drops_ready_prefetches():
    m = ReadyTimeExpertCacheManager(capacity=0, service_us_per_issue=1.0, queue_batch_size=1,
                                    queue_deadline_us=5.0)
    assert m.issue_prefetch(0, 1, arrival_us=0.0) is True
    m.finish()
    s = m.snapshot()
    assert (s.resident_count, s.issued_fetch_count, s.evicted_before_use_count) == (0, 1, 1)


def test_ready_time_underfilled_batch_flushes_at_deadline():
    m = ReadyTimeExpertCacheManager(capacity=2, service_us_per_issue=1.0, queue_batch_size=2,
                                    queue_deadline_us=5.0)
    assert m.issue_prefetch(0, 1, arrival_us=0.0) is True
    assert m.demand(0, 1, arrival_us=0.0) is False
    m.finish()
    s = m.snapshot()
    assert (s.queue_batch_count, s.queue_service_us, s.queue_total_span_us, s.demand_miss_count,
            s.ready_late_miss_count, s.late_completion_unused_count) == (1, 1.0, 6.0, 1, 1, 1)


def test_ready_time_rejects_non_finite_and_clamps():
    for kw in ({"service_us_per_issue": math.inf}, {"service_us_per_batch": math.nan},
               {"queue_deadline_us": math.inf}):
        with pytest.raises(ValueError):
            ReadyTimeExpertCacheManager(capacity=2, **kw)
    m = ReadyTimeExpertCacheManager(capacity=2, service_us_per_issue=-1.0, queue_batch_size=0,
                                    queue_deadline_us=-3.0)
    s = m.snapshot()
    assert (m.service_us_per_issue, s.queue_batch_size, s.queue_deadline_us) == (0.0, 1, 0.0)
    rc = _lib.load().moe_ready_cache_create_v1(1, 4, math.nan, 0.0, 1, 0.0, None)
    assert rc == _lib.MOE_ERR_NULL  # the NULL handle is checked first
    import ctypes
    h = ctypes.c_uint64()
    assert _lib.load().moe_ready_cache_create_v1(1, 4, math.nan, 0.0, 1, 0.0, ctypes.byref(h)) == _lib.MOE_ERR_SHAPE
    assert _lib.load().moe_ready_cache_create_v1(7, 4, 0.0, 0.0, 1, 0.0, ctypes.byref(h)) == _lib.MOE_ERR_UNSUPPORTED


def _oracle_snapshot(o: ReadyTimeCounters) -> dict:
    return o.stats()


@pytest.mark.parametrize("seed", range(6))
def test_ready_time_random_sequences_match_the_oracle(seed):
    rng = random.Random(seed)
    cap = rng.choice((0, 1, 3, 8, 24))
    per_issue = rng.choice((0.0, 1.0, 7.5, 40.0))
    per_batch = rng.choice((0.0, 3.0))
    batch = rng.choice((1, 2, 4))
    deadline = rng.choice((0.0, 5.0, 50.0))
    m = ReadyTimeExpertCacheManager(capacity=cap, service_us_per_issue=per_issue,
                                    service_us_per_batch=per_batch, queue_batch_size=batch,
                                    queue_deadline_us=deadline)
    o = ReadyTimeCounters(cap, per_issue, per_batch, batch, deadline)
    t = 0.0
    for _ in range(600):
        t += rng.choice((0.0, 0.5, 2.0, 9.0))
        layer = rng.randrange(3)
        r = rng.random()
        if r < 0.45:
            experts = [rng.randrange(16) for _ in range(rng.randint(1, 4))]
            got = [m.issue_prefetch(layer, e, arrival_us=t) for e in experts]
            want = [o.issue_prefetch(layer, e, t) for e in experts]
        elif r < 0.9:
            experts = [rng.randrange(16) for _ in range(rng.randint(1, 3))]
            got = m.demand_many(layer, experts, arrival_us=t)
            want = [o.demand(layer, e, t) for e in experts]
        else:
            m.advance_to(t)
            o.advance_to(t)
            got = want = []
        assert got == want
    m.finish()
    o.finish()
    s = m.snapshot().as_dict()
    for k, v in _oracle_snapshot(o).items():
        assert s[k] == pytest.approx(v, abs=1e-9), k


@pytest.mark.parametrize("seed", range(3))
def test_controlled_random_sequences_match_the_oracle(seed):
    rng = random.Random(100 + seed)
    cap = rng.choice((0, 2, 5, 16))
    m = ControlledExpertCacheManager(capacity=cap)
    o = LruCounters(cap)
    for _ in range(800):
        layer, e = rng.randrange(4), rng.randrange(12)
        if rng.random() < 0.5:
            assert m.issue_prefetch(layer, e) == o.issue_prefetch(layer, e)
        else:
            assert m.demand(layer, e) == o.demand(layer, e)
    s = m.snapshot()
    assert (s.issued_fetch_count, s.used_fetch_count, s.unused_fetch_count, s.demand_count,
            s.demand_hit_count, s.demand_miss_count, s.evicted_before_use_count,
            s.resident_count) == (o.issued, o.used, o.unused(), o.demand_count, o.hits, o.misses,
                                  o.evicted_before_use, len(o.cache))
