"""Pins the oracle align/sort (oracle/moe_ref.py:align_block_padded)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_ref


def test_reference_kat_format():
    # format of tests/test_vllm_descriptor_mapping_assertion.py:1012-1085: topk_ids [[1,2,3]],
    # BLOCK_M=4 -> 3 blocks, num_tokens_post_padded 12, sentinel 3 = topk_ids.numel(), one
    # routed slot per block. The reference orders blocks by a layer prior ([2, 1, 3]); this
    # build's stable order is experts ascending.
    sorted_ids, eids, ntpp = moe_ref.align_block_padded(np.array([[1, 2, 3]]), 8, 4)
    assert ntpp == 12
    assert eids.tolist() == [1, 2, 3]
    assert sorted_ids.reshape(3, 4).tolist() == [[0, 3, 3, 3], [1, 3, 3, 3], [2, 3, 3, 3]]


def _brute(ids: np.ndarray, E: int, BM: int, has_shared: bool):
    T, k = ids.shape
    slots = [(int(ids[t, i]), t * k + i) for t in range(T) for i in range(k)]
    if has_shared:
        slots += [(E, T * k + t) for t in range(T)]
    n = len(slots)
    out, eids = [], []
    for e in range(E + (1 if has_shared else 0)):
        mine = sorted(f for ee, f in slots if ee == e)
        if not mine:
            continue
        pad = -(-len(mine) // BM) * BM
        out += mine + [n] * (pad - len(mine))
        eids += [e] * (pad // BM)
    return out, eids, len(out)


@pytest.mark.parametrize("T,k,E,BM,shared", [(1, 8, 256, 16, False), (5, 4, 16, 4, True),
                                              (64, 8, 256, 16, False), (33, 8, 32, 128, True),
                                              (0, 8, 16, 16, False)])
def test_align_matches_brute_force(T, k, E, BM, shared):
    rng = np.random.default_rng(T * 131 + k)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]) if T else np.zeros((0, k), np.int64)
    s, e, n = moe_ref.align_block_padded(ids, E, BM, has_shared=shared)
    bs, be, bn = _brute(ids, E, BM, shared)
    assert n == bn and s.tolist() == bs and e.tolist() == be
    # invariants: a permutation of all slots plus sentinels; single-expert blocks; ntpp % BM == 0
    n_slots = T * k + (T if shared else 0)
    assert sorted(x for x in s.tolist() if x < n_slots) == list(range(n_slots))
    assert n % BM == 0


def test_capacity_bound_holds():
    rng = np.random.default_rng(9)
    for _ in range(50):
        T, k, E, BM = int(rng.integers(1, 80)), 8, 256, int(rng.choice([1, 4, 16, 128]))
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
        _, eids, ntpp = moe_ref.align_block_padded(ids, E, BM)
        assert ntpp // BM <= moe_ref.max_blocks(T * k, E, BM)
