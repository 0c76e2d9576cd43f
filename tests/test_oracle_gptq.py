"""Pins the oracle's unpack/dequant (oracle/gptq_ref.py) before it is trusted.

Checks: the reference's own known-answer tests (tests/test_gptq_unpack.py:17-82 restated),
torch's RNE bf16 cast as a library routine, brute force on tiny inputs, special nibble patterns,
and a planted-mistake check showing a wrong nibble order fails the KAT.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import gptq_ref


def test_unpack_rows_and_cols_round_trip_4bit():
    # reference KAT: tests/test_gptq_unpack.py:41-46
    row_values = (np.arange(16 * 8, dtype=np.int32).reshape(16, 8) % 16)
    col_values = (np.arange(2 * 16, dtype=np.int32).reshape(2, 16) % 16)
    assert np.array_equal(gptq_ref.unpack_rows(gptq_ref.pack_rows(row_values)), row_values)
    assert np.array_equal(gptq_ref.unpack_cols(gptq_ref.pack_cols(col_values)), col_values)


def test_unpack_nibble_positions_and_sign_bit():
    # nibble j of qweight[r, n] is W[8r + j, n]; -1 (all bits set) unpacks to all 15
    packed = np.array([[0x76543210, -1, np.int32(-0x80000000)]], dtype=np.int32)
    w = gptq_ref.unpack_rows(packed)
    assert w[:, 0].tolist() == [0, 1, 2, 3, 4, 5, 6, 7]
    assert w[:, 1].tolist() == [15] * 8
    assert w[:, 2].tolist() == [0] * 7 + [8]
    z = gptq_ref.unpack_cols(np.array([[0x76543210]], dtype=np.int32))
    assert z[0].tolist() == [0, 1, 2, 3, 4, 5, 6, 7]


def _kat_tensors():
    # reference KAT: tests/test_gptq_unpack.py:49-77
    int_weight = (np.arange(16 * 8, dtype=np.int32).reshape(16, 8) % 16)
    zeros = np.stack([np.full(8, 2, np.int32), np.full(8, 5, np.int32)])
    scales = np.stack([np.linspace(0.25, 1.0, 8, dtype=np.float32),
                       np.linspace(1.0, 1.75, 8, dtype=np.float32)]).astype(np.float16)
    g_idx = np.array([0] * 8 + [1] * 8, dtype=np.int32)
    return int_weight, zeros, scales, g_idx


def test_dequant_matches_reference_kat():
    int_weight, zeros, scales, g_idx = _kat_tensors()
    got = gptq_ref.dequant_f32(gptq_ref.pack_rows(int_weight), gptq_ref.pack_cols(zeros),
                               scales.view(np.uint16), g_idx, group_size=8)
    expected = ((int_weight.astype(np.float32) - zeros.astype(np.float32)[g_idx])
                * scales.astype(np.float32)[g_idx]).T
    assert got.shape == (8, 16)
    assert np.array_equal(got, expected)


def test_planted_nibble_order_mistake_fails_kat():
    # a plausible bug (reversed nibble order inside an int32) must be caught by the KAT
    int_weight, zeros, scales, g_idx = _kat_tensors()
    packed = gptq_ref.pack_rows(int_weight)
    wrong = gptq_ref.unpack_rows(packed)[::-1].copy()  # reversed k order
    right = gptq_ref.unpack_rows(packed)
    assert not np.array_equal(wrong, right)
    assert not np.array_equal(wrong, int_weight)


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.4e38, 1e-40, -1e-40,
                  1.00390625, 1.01171875, 1.0078125], dtype=np.float32),  # exact ties
    ]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(gptq_ref.f32_to_bf16_bits(x), ref)
    nan = gptq_ref.f32_to_bf16_bits(np.array([np.nan], dtype=np.float32))
    assert np.isnan(gptq_ref.bf16_bits_to_f32(nan))[0]


def test_dequant_brute_force_tiny_and_exact_product():
    rng = np.random.default_rng(1)
    K, N, G = 16, 8, 8
    q = rng.integers(0, 16, (K, N)).astype(np.int32)
    z = rng.integers(0, 16, (K // G, N)).astype(np.int32)
    s = rng.uniform(0.002, 0.02, (K // G, N)).astype(np.float16)
    got = gptq_ref.dequant_bf16_bits(gptq_ref.pack_rows(q), gptq_ref.pack_cols(z), s.view(np.uint16),
                                     group_size=G)
    for n in range(N):
        for k in range(K):
            exact = (int(q[k, n]) - int(z[k // G, n])) * float(s[k // G, n])  # python float64
            assert np.float32(exact) == exact  # the fp32 product is exact
            want = torch.tensor(exact, dtype=torch.float32).to(torch.bfloat16).view(torch.int16).item() & 0xFFFF
            assert int(got[n, k]) == want
