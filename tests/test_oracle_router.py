"""Pins the oracle router (oracle/moe_ref.py): canonical logit order, top-k tie rule, weights."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import gptq_ref, moe_ref


def _bf16(rng, shape, scale=1.0):
    return gptq_ref.f32_to_bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))


def test_canonical_dot_matches_pure_python_lane_emulation():
    rng = np.random.default_rng(2)
    K = 1024
    x = gptq_ref.bf16_bits_to_f32(_bf16(rng, (2, K)))
    w = gptq_ref.bf16_bits_to_f32(_bf16(rng, (3, K), 0.02))
    got = moe_ref.canonical_dot_rows(x, w)
    for t in range(2):
        for e in range(3):
            part = []
            for lane in range(64):
                acc = np.float32(0.0)
                q = lane
                while q < K // 8:
                    for i in range(8):
                        k = 8 * q + i
                        acc = np.float32(acc + np.float32(x[t, k] * w[e, k]))
                    q += 64
                part.append(acc)
            m = 32
            vals = part
            while m >= 1:
                vals = [np.float32(vals[l] + vals[l ^ m]) for l in range(64)]
                m //= 2
            assert got[t, e] == vals[0]


def test_canonical_dot_close_to_float64():
    rng = np.random.default_rng(3)
    x = gptq_ref.bf16_bits_to_f32(_bf16(rng, (8, 2048)))
    w = gptq_ref.bf16_bits_to_f32(_bf16(rng, (16, 2048), 0.02))
    got = moe_ref.canonical_dot_rows(x, w)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.max(np.abs(got - ref)) < 1e-4


def test_topk_tie_rule_and_all_equal():
    logits = np.zeros((1, 16), dtype=np.float32)
    ids = moe_ref.stable_topk(logits, 8)
    assert ids.tolist() == [list(range(8))]
    w = moe_ref.renorm_weights(logits, ids)
    assert np.allclose(w, 1.0 / 8)
    # torch.topk(tensor([0,1,1,1,.5]),2) may return [1,3]; the stable rule gives [1,2]
    ids = moe_ref.stable_topk(np.array([[0, 1, 1, 1, 0.5]], dtype=np.float32), 2)
    assert ids.tolist() == [[1, 2]]


def test_topk_matches_brute_force_sort():
    rng = np.random.default_rng(4)
    logits = np.round(rng.standard_normal((50, 32)) * 4).astype(np.float32)  # many ties
    ids = moe_ref.stable_topk(logits, 8)
    for t in range(50):
        order = sorted(range(32), key=lambda e: (-float(logits[t, e]), e))[:8]
        assert ids[t].tolist() == order


def test_weights_equal_softmax_topk_renorm_and_sum_to_one():
    # reference semantics: p = softmax(logits); top-k; w = p_top / max(sum, 1e-20)
    # (tracing/vllm_router_trace.py:4216-4221); weights sum to 1 (tests/test_mtp_extra_tensors.py:69)
    rng = np.random.default_rng(5)
    logits = (rng.standard_normal((40, 256)) * 2).astype(np.float32)
    ids = moe_ref.stable_topk(logits, 8)
    w = moe_ref.renorm_weights(logits, ids)
    p = np.exp(logits.astype(np.float64) - logits.max(axis=1, keepdims=True))
    p = p / p.sum(axis=1, keepdims=True)
    sel = np.take_along_axis(p, ids.astype(np.int64), axis=1)
    ref = sel / np.maximum(sel.sum(axis=1, keepdims=True), 1e-20)
    assert np.max(np.abs(w - ref)) < 1e-6
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)


def test_one_dominant_logit():
    logits = np.full((1, 64), -5.0, dtype=np.float32)
    logits[0, 37] = 30.0
    ids, = moe_ref.stable_topk(logits, 4)
    assert ids[0] == 37 and ids[1:].tolist() == [0, 1, 2]
    w = moe_ref.renorm_weights(logits, ids[None])
    assert w[0, 0] == pytest.approx(1.0, abs=1e-12)
