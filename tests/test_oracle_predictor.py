"""Pins the predictor oracle (per-layer bf16 MLP hidden -> inner SiLU -> experts, top-k).

The oracle's canonical-order products are checked against float64 matmuls, its SiLU against
torch's, its bf16 rounding against torch's bf16 cast, and its top-k against a brute-force sort;
a dropped SiLU, a transposed weight or a head mix-up each fail one of these.
"""

import numpy as np
import torch
import torch.nn.functional as F

from oracle import gptq_ref, moe_ref


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _case(seed=0, T=2, L=3, H=64, D=32, E=24):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(T, H, generator=g)
    w1 = torch.randn(L, D, H, generator=g) * 0.2
    w2 = torch.randn(L, E, D, generator=g) * 0.2
    return _bf16_bits(h), _bf16_bits(w1), _bf16_bits(w2)


def test_predictor_matches_float64_path():
    h_bits, w1_bits, w2_bits = _case()
    ids, logits = moe_ref.predictor_ref(h_bits, w1_bits, w2_bits, top_k=5)
    h = torch.from_numpy(gptq_ref.bf16_bits_to_f32(h_bits)).double()
    L = w1_bits.shape[0]
    assert ids.shape == (L, h.shape[0], 5) and logits.shape == (L, h.shape[0], w2_bits.shape[1])
    for l in range(L):
        w1 = torch.from_numpy(gptq_ref.bf16_bits_to_f32(w1_bits[l])).double()
        w2 = torch.from_numpy(gptq_ref.bf16_bits_to_f32(w2_bits[l])).double()
        a = F.silu(h @ w1.T).float().to(torch.bfloat16).double()
        ref = a @ w2.T
        np.testing.assert_allclose(logits[l], ref.numpy(), rtol=2e-2, atol=2e-3)
        # brute-force top-k on the oracle's own logits (value desc, id asc)
        for t in range(h.shape[0]):
            order = sorted(range(logits.shape[2]), key=lambda e: (-float(logits[l, t, e]), e))
            assert list(ids[l, t]) == order[:5]


def test_heads_are_independent():
    """Head l depends only on w1[l], w2[l]: swapping heads swaps the outputs."""
    h_bits, w1_bits, w2_bits = _case(seed=1)
    ids, logits = moe_ref.predictor_ref(h_bits, w1_bits, w2_bits, top_k=4)
    ids_r, logits_r = moe_ref.predictor_ref(h_bits, w1_bits[::-1].copy(), w2_bits[::-1].copy(), top_k=4)
    np.testing.assert_array_equal(ids_r, ids[::-1])
    np.testing.assert_array_equal(logits_r, logits[::-1])


def test_silu_is_applied_once_and_rounded_to_bf16():
    """With w2 = identity rows the logits are the bf16-rounded SiLU activations themselves."""
    T, H, D = 2, 16, 8
    g = torch.Generator().manual_seed(3)
    h = torch.randn(T, H, generator=g)
    w1 = torch.randn(1, D, H, generator=g) * 0.3
    w2 = torch.eye(D).reshape(1, D, D)
    ids, logits = moe_ref.predictor_ref(_bf16_bits(h), _bf16_bits(w1), _bf16_bits(w2), top_k=D)
    z1 = moe_ref.canonical_dot_rows(gptq_ref.bf16_bits_to_f32(_bf16_bits(h)),
                                    gptq_ref.bf16_bits_to_f32(_bf16_bits(w1[0])))
    want = F.silu(torch.from_numpy(z1)).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(logits[0], want)
