"""Pins the oracle expert MLP / top-k sum / layer (oracle/moe_ref.py)."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import gptq_ref, moe_ref


def test_single_expert_matches_manual_formula():
    # restates tests/test_gptq_unpack.py:85-124
    wg = torch.tensor([[0.5, -0.25, 0.75, 0.0], [0.0, 0.5, -0.5, 1.0], [1.0, 0.0, 0.25, -0.75]])
    wu = torch.tensor([[0.25, 0.5, 0.0, -0.25], [0.75, -0.5, 0.5, 0.0], [-0.25, 0.25, 1.0, 0.5]])
    wd = torch.tensor([[0.5, 0.25, -0.5], [0.0, 0.75, 0.25], [-0.25, 0.5, 0.5], [1.0, -0.5, 0.0]])
    x = torch.randn(10, 4, generator=torch.Generator().manual_seed(0))
    expected = F.linear(F.silu(F.linear(x, wg)) * F.linear(x, wu), wd)
    assert torch.allclose(moe_ref.expert_mlp_f32(x, wg, wu, wd), expected)


def _layer_np(E, H, I, seed):
    rng = np.random.default_rng(seed)
    d = {"group_size": 128}
    for proj, (k, n) in (("gate_proj", (H, I)), ("up_proj", (H, I)), ("down_proj", (I, H))):
        d[f"{proj}.qweight"] = rng.integers(-2**31, 2**31, (E, k // 8, n), dtype=np.int64).astype(np.int32)
        d[f"{proj}.qzeros"] = rng.integers(-2**31, 2**31, (E, k // 128, n // 8), dtype=np.int64).astype(np.int32)
        d[f"{proj}.scales"] = rng.uniform(0.002, 0.02, (E, k // 128, n)).astype(np.float16).view(np.uint16)
    return d


def test_topk_sum_weighted_and_order_preserving():
    # restates tests/test_gptq_unpack.py:127-153 on quantised experts: out = sum_i w_i * expert_i(x)
    E, H, I = 8, 256, 128
    layer = _layer_np(E, H, I, 0)
    rng = np.random.default_rng(1)
    x_bits = gptq_ref.f32_to_bf16_bits(rng.standard_normal((3, H)).astype(np.float32))
    ids = np.array([[7, 3]] * 3, dtype=np.int32)
    w = np.array([[0.25, 0.75]] * 3, dtype=np.float32)
    out = moe_ref.moe_layer_f32(x_bits, ids, w, layer)
    x = torch.from_numpy(gptq_ref.bf16_bits_to_f32(x_bits))
    e7 = moe_ref.expert_mlp_f32(x, *moe_ref.dequant_expert(layer, 7))
    e3 = moe_ref.expert_mlp_f32(x, *moe_ref.dequant_expert(layer, 3))
    assert np.allclose(out, (0.25 * e7 + 0.75 * e3).numpy(), rtol=1e-5, atol=1e-4)


def test_f32_oracle_agrees_with_reference_bf16_flow():
    # two restatements (fp32 accumulation vs the reference's bf16 F.linear flow,
    # extra_tensors.py:544-598) must agree to bf16 accuracy
    E, H, I, T, k = 16, 512, 256, 12, 4
    layer = _layer_np(E, H, I, 2)
    rng = np.random.default_rng(3)
    x_bits = gptq_ref.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    rw_bits = gptq_ref.f32_to_bf16_bits((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    ids, w, _ = moe_ref.router_topk(x_bits, rw_bits, k)
    ref32 = moe_ref.moe_layer_f32(x_bits, ids, w, layer)
    experts = {}
    for e in np.unique(ids):
        experts[int(e)] = tuple(t.to(torch.bfloat16) for t in moe_ref.dequant_expert(layer, int(e)))
    x = torch.from_numpy(gptq_ref.bf16_bits_to_f32(x_bits)).to(torch.bfloat16)
    out16 = moe_ref.moe_tokens_bf16(x, torch.from_numpy(ids).long(), torch.from_numpy(w), experts)
    assert moe_ref.rel_err(out16.float().numpy(), ref32) < 2e-2


def test_torch_stack_dequant_matches_numpy_restatement():
    layer = _layer_np(3, 256, 128, 4)
    for proj in ("gate_proj", "down_proj"):
        got = moe_ref.dequant_stack_torch(torch.from_numpy(layer[f"{proj}.qweight"]),
                                          torch.from_numpy(layer[f"{proj}.qzeros"]),
                                          torch.from_numpy(layer[f"{proj}.scales"].view(np.float16)))
        for e in range(3):
            want = gptq_ref.dequant_bf16_bits(layer[f"{proj}.qweight"][e], layer[f"{proj}.qzeros"][e],
                                              layer[f"{proj}.scales"][e])
            assert np.array_equal(got[e].view(torch.int16).numpy().view(np.uint16), want)


def test_rel_err_metric():
    ref = np.array([1.0, -4.0, 2.0])
    assert abs(moe_ref.rel_err(ref + np.array([0.0, 0.04, 0.0]), ref) - 0.01) < 1e-12
