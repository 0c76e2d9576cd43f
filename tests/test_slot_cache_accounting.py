"""Slot-cache accounting of the C library (dry run: no HIP calls) against the LRU counter oracle.

Reference semantics: src/mtp_expert_prefetch/runtime/cache_manager.py:208-279; the reference's
own cases are tests/test_cache_manager.py:21-160 (LRU hit/miss, evicted-before-use, capacity 0,
dedup of resident issues). The library keeps one LRU of `slots_per_layer` entries per layer, so a
one-layer cache must match the reference's single LRU exactly, and a multi-layer cache must match
one oracle instance per layer.
"""

import random

import pytest

from mtp_amd import _lib
from mtp_amd.offload import SlotCache, blob_layout
from oracle.cache_ref import LruCounters


def _lib_or_skip():
    try:
        return _lib.load()
    except RuntimeError as exc:  # library not built in this checkout
        pytest.skip(str(exc))


def _oracle_stats(oracles: list[LruCounters]) -> dict[str, int]:
    return {
        "issued_fetch_count": sum(o.issued for o in oracles),
        "used_fetch_count": sum(o.used for o in oracles),
        "unused_fetch_count": sum(o.unused() for o in oracles),
        "demand_count": sum(o.demand_count for o in oracles),
        "demand_hit_count": sum(o.hits for o in oracles),
        "demand_miss_count": sum(o.misses for o in oracles),
        "evicted_before_use_count": sum(o.evicted_before_use for o in oracles),
        "resident_count": sum(len(o.cache) for o in oracles),
    }


def _check(cache: SlotCache, oracles: list[LruCounters]) -> None:
    got = cache.stats()
    want = _oracle_stats(oracles)
    for k, v in want.items():
        assert got[k] == v, (k, got[k], v)
    for layer, o in enumerate(oracles):
        resident = {e for (l, e) in o.cache if l == layer}
        for e in range(cache.num_experts):
            assert (cache.slot_of(layer, e) >= 0) == (e in resident), (layer, e)


def test_reference_lru_cases():
    """The reference's hand cases (test_cache_manager.py:21-160) on one layer."""
    _lib_or_skip()
    with SlotCache(1, 8, 2, 16, dry_run=True) as c:
        o = [LruCounters(2)]
        assert c.prefetch(0, [1]) == 1 and o[0].issue_prefetch(0, 1)
        assert c.prefetch(0, [1]) == 0 and not o[0].issue_prefetch(0, 1)  # resident: no issue
        assert c.demand(0, [1]) == 1 and o[0].demand(0, 1)                 # used prefetch
        assert c.demand(0, [2]) == 0 and not o[0].demand(0, 2)             # miss inserts
        c.layer_done(0)                                                     # kernels enqueued
        c.prefetch(0, [3]); o[0].issue_prefetch(0, 3)                       # evicts 1 (LRU)
        c.prefetch(0, [4]); o[0].issue_prefetch(0, 4)                       # evicts 2
        c.prefetch(0, [5]); o[0].issue_prefetch(0, 5)                       # evicts 3 unused
        _check(c, o)
        assert c.stats()["evicted_before_use_count"] == 1


def test_capacity_zero_counts_every_prefetch_as_evicted():
    _lib_or_skip()
    with SlotCache(1, 4, 0, 16, dry_run=True) as c:
        o = [LruCounters(0)]
        for e in (0, 1, 1, 2):
            c.prefetch(0, [e]); o[0].issue_prefetch(0, e)
            c.demand(0, [e]); o[0].demand(0, e)
        _check(c, o)
        assert c.stats()["resident_count"] == 0


@pytest.mark.parametrize("layers,experts,slots,seed", [(1, 16, 4, 0), (1, 32, 8, 1), (3, 24, 5, 2),
                                                       (2, 256, 64, 3)])
def test_random_sequences_match_oracle(layers, experts, slots, seed):
    _lib_or_skip()
    rng = random.Random(seed)
    with SlotCache(layers, experts, slots, 1 << 20, dry_run=True) as c:
        oracles = [LruCounters(slots) for _ in range(layers)]
        for step in range(600):
            layer = rng.randrange(layers)
            n = rng.randrange(0, min(slots, 8) + 1)
            ids = [rng.randrange(experts) for _ in range(n)]
            if rng.random() < 0.5:
                issued = c.prefetch(layer, ids)
                assert issued == sum(oracles[layer].issue_prefetch(layer, e) for e in ids)
            else:
                hits = c.demand(layer, ids)
                assert hits == sum(oracles[layer].demand(layer, e) for e in ids)
                c.layer_done(layer)  # the layer's kernels are enqueued
            if step % 50 == 0:
                _check(c, oracles)
        _check(c, oracles)


def test_prefetch_never_evicts_slots_of_the_latest_demand():
    """Between a demand and layer_done the demanded slots may still be read by kernels that are
    not enqueued yet: a prefetch takes other slots, or skips when only pinned slots remain."""
    _lib_or_skip()
    with SlotCache(1, 16, 3, 16, dry_run=True) as c:
        c.demand(0, [1, 2])
        s1, s2 = c.slot_of(0, 1), c.slot_of(0, 2)
        assert c.prefetch(0, [5]) == 1          # the free slot
        assert c.prefetch(0, [6]) == 1          # evicts 5 (the only unpinned), not 1 or 2
        assert c.slot_of(0, 5) == -1 and c.slot_of(0, 6) >= 0
        assert (c.slot_of(0, 1), c.slot_of(0, 2)) == (s1, s2)
        c.demand(0, [1, 2, 6])                  # every slot pinned
        assert c.prefetch(0, [7]) == 0
        st = c.stats()
        assert st["prefetch_skipped_pinned_count"] == 1 and c.slot_of(0, 7) == -1
        assert st["evicted_before_use_count"] == 1          # 5 was evicted unused
        c.layer_done(0)
        assert c.prefetch(0, [7]) == 1          # LRU again: evicts 1
        assert c.slot_of(0, 1) == -1 and c.slot_of(0, 7) >= 0
        # the next demand of the layer replaces the pins of the previous one
        c.demand(0, [2])
        assert c.prefetch(0, [8]) == 1 and c.slot_of(0, 2) >= 0
        with pytest.raises(_lib.MoeLibraryError):
            c.layer_done(1)


def test_bad_arguments_raise():
    _lib_or_skip()
    with SlotCache(2, 8, 2, 16, dry_run=True) as c:
        with pytest.raises(_lib.MoeLibraryError):
            c.prefetch(2, [0])
        with pytest.raises(_lib.MoeLibraryError):
            c.demand(0, [8])
        with pytest.raises(IndexError):
            c.slot_of(0, 9)
        # a failed call leaves the counters untouched
        assert c.stats()["issued_fetch_count"] == 0 and c.stats()["demand_count"] == 0
    with pytest.raises(_lib.MoeLibraryError):
        SlotCache(1, 8, 2, 15, dry_run=True)      # blob size not a multiple of 16
    with pytest.raises(_lib.MoeLibraryError):
        SlotCache(1, 8, 2, 16, dry_run=False)     # live cache without pools


def test_blob_layout_qwen3_shape():
    pieces, blob = blob_layout(2048, 512, 128)
    assert blob == 1_634_304
    offsets = {(p.proj, p.kind): p.offset for p in pieces}
    assert offsets[("gate", "qweight")] == 0
    assert offsets[("gate", "qzeros")] == 524_288
    assert offsets[("gate", "scales")] == 528_384
    assert offsets[("up", "qweight")] == 544_768
    assert offsets[("down", "qweight")] == 1_089_536
    assert offsets[("down", "scales")] == 1_617_920
