"""Pins the oracle's shared-expert gate and the shared branch of the layer oracle.

Reference: mtp/extra_tensors.py:596-597 (out += sigmoid(x . w_g) * shared_expert(x)) and the
vLLM hook restated at tracing/vllm_router_trace.py:4038-4089. The checks are closed forms
(w_g = 0 gives exactly 0.5, saturation at large |x . w_g|), an independent float64 evaluation,
and, for the layer, a hand-summed routed + g * shared and the reference's own bf16 dtype flow.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import gptq_ref, moe_ref
from tests.test_oracle_moe import _layer_np


def _bits(a: np.ndarray) -> np.ndarray:
    return gptq_ref.f32_to_bf16_bits(a.astype(np.float32))


def test_shared_gate_zero_weight_is_one_half():
    rng = np.random.default_rng(0)
    x = _bits(rng.standard_normal((5, 256)))
    g = moe_ref.shared_gate(x, _bits(np.zeros(256)))
    assert g.dtype == np.float32
    assert np.array_equal(g, np.full(5, 0.5, dtype=np.float32))


def test_shared_gate_saturates_with_the_sign_of_the_dot():
    H = 128
    x = _bits(np.ones((2, H)))
    x[1] = _bits(-np.ones(H))
    w = _bits(np.full(H, 1.0))  # x . w = +128 for row 0, -128 for row 1
    g = moe_ref.shared_gate(x, w)
    assert g[0] == np.float32(1.0)
    assert 0.0 <= g[1] < 1e-30
    # a small positive dot gives a gate just above one half, a negative one just below
    w_small = _bits(np.full(H, 1.0 / 1024))
    g2 = moe_ref.shared_gate(x, w_small)  # dots +0.125 and -0.125
    assert 0.5 < g2[0] < 0.54 and 0.46 < g2[1] < 0.5
    assert abs((g2[0] - 0.5) + (g2[1] - 0.5)) < 1e-7


def test_shared_gate_matches_float64_sigmoid():
    rng = np.random.default_rng(1)
    T, H = 32, 2048
    x = _bits(rng.standard_normal((T, H)))
    w = _bits(rng.standard_normal(H) * 0.02)
    xf = gptq_ref.bf16_bits_to_f32(x).astype(np.float64)
    wf = gptq_ref.bf16_bits_to_f32(w).astype(np.float64)
    want = 1.0 / (1.0 + np.exp(-(xf @ wf)))
    got = moe_ref.shared_gate(x, w)
    # the oracle's fp32 canonical-order dot differs from the float64 dot by rounding only
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=0)
    # the gate follows row t of x: permuting the tokens permutes the gates
    perm = rng.permutation(T)
    assert np.array_equal(moe_ref.shared_gate(x[perm], w), got[perm])


def test_layer_shared_branch_is_routed_plus_gated_shared():
    E, H, I, T = 8, 256, 128, 6
    layer = _layer_np(E, H, I, 10)
    shared = _layer_np(1, H, I, 11)
    rng = np.random.default_rng(12)
    x = _bits(rng.standard_normal((T, H)))
    ids = np.stack([rng.choice(E, 2, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.1, 0.9, (T, 2)).astype(np.float32)
    g = rng.uniform(0.05, 0.95, T).astype(np.float32)

    routed = moe_ref.moe_layer_f32(x, ids, w, layer)
    full = moe_ref.moe_layer_f32(x, ids, w, layer, shared=shared, shared_gate_values=g)

    # by hand: dequantise the shared expert (bit-exact bf16 weights) and evaluate it in float64
    xs = gptq_ref.bf16_bits_to_f32(x).astype(np.float64)
    deq = [gptq_ref.bf16_bits_to_f32(gptq_ref.dequant_bf16_bits(
        shared[f"{p}.qweight"][0], shared[f"{p}.qzeros"][0], shared[f"{p}.scales"][0])).astype(np.float64)
        for p in ("gate_proj", "up_proj", "down_proj")]
    gate, up = xs @ deq[0].T, xs @ deq[1].T
    y_shared = ((gate / (1.0 + np.exp(-gate))) * up) @ deq[2].T
    want = routed.astype(np.float64) + g.astype(np.float64)[:, None] * y_shared
    assert moe_ref.rel_err(full, want) < 1e-5
    # the shared expert is the slot set's extra row: zero gates leave the routed sum unchanged
    same = moe_ref.moe_layer_f32(x, ids, w, layer, shared=shared,
                                 shared_gate_values=np.zeros(T, dtype=np.float32))
    assert np.array_equal(same, routed)


def test_layer_shared_branch_agrees_with_reference_bf16_flow():
    """The fp32 oracle with the shared expert against the reference's own bf16 dtype flow
    (extra_tensors.py:544-598, including its sigmoid(F.linear(x, w_g)) gate)."""
    E, H, I, T, k = 16, 512, 256, 10, 4
    layer = _layer_np(E, H, I, 20)
    shared = _layer_np(1, H, I, 21)
    rng = np.random.default_rng(22)
    x = _bits(rng.standard_normal((T, H)))
    rw = _bits(rng.standard_normal((E, H)) * 0.02)
    gw = _bits(rng.standard_normal(H) * 0.05)
    ref32, ids, w, sg = moe_ref.moe_layer_ref(x, rw, layer, top_k=k, shared=shared,
                                              shared_gate_w_bits=gw)
    experts = {int(e): tuple(t.to(torch.bfloat16) for t in moe_ref.dequant_expert(layer, int(e)))
               for e in np.unique(ids)}
    shared_w = tuple(t.to(torch.bfloat16) for t in moe_ref.dequant_expert(shared, 0))
    xt = torch.from_numpy(gptq_ref.bf16_bits_to_f32(x)).to(torch.bfloat16)
    gwt = torch.from_numpy(gptq_ref.bf16_bits_to_f32(gw)).to(torch.bfloat16).view(1, H)
    out16 = moe_ref.moe_tokens_bf16(xt, torch.from_numpy(ids).long(), torch.from_numpy(w), experts,
                                    shared=shared_w, shared_gate_w=gwt)
    assert moe_ref.rel_err(out16.float().numpy(), ref32) < 2e-2
    # the gate itself: bf16 F.linear + sigmoid against the oracle's fp32 gate
    g16 = torch.sigmoid(F.linear(xt, gwt)).float().numpy()[:, 0]
    np.testing.assert_allclose(g16, sg, atol=8e-3)
    # and a planted sign error in the gate would be caught by this comparison
    bad = moe_ref.moe_layer_f32(x, ids, w, layer, shared=shared, shared_gate_values=1.0 - sg)
    assert moe_ref.rel_err(out16.float().numpy(), bad) > 2e-2
