"""Pins the AWQ layouts of the oracle (oracle/awq_ref.py) and their repack into GPTQ.

wna16: vLLM's int4 fused-MoE layout as the reference restates it
(tracing/vllm_wna16_group_plan.py:394-470: b_shifter = (k % 2) * 4 on byte k // 2 of row n,
b_zp_shifter = (n % 2) * 4 on byte n // 2 of group g, zero 8 without zero points, dequant
(q - z) * s). awq: the AutoAWQ GEMM packing order [0, 2, 4, 6, 1, 3, 5, 7] along N.
"""

from __future__ import annotations

import numpy as np

from oracle import awq_ref, gptq_ref


def test_wna16_byte_layout_known_answers():
    b = np.zeros((2, 4), dtype=np.uint8)  # N = 2, K = 8
    b[0, 0] = 0x21   # k = 0 -> 1 (low nibble), k = 1 -> 2 (high nibble), column 0
    b[1, 3] = 0xF7   # k = 6 -> 7, k = 7 -> 15, column 1
    q = awq_ref.wna16_unpack(b)
    assert q.shape == (8, 2)
    assert (q[0, 0], q[1, 0], q[6, 1], q[7, 1]) == (1, 2, 7, 15)
    assert q.sum() == 1 + 2 + 7 + 15
    zp = np.array([[0xA5]], dtype=np.uint8)  # N = 2, one group
    z = awq_ref.wna16_zeros_unpack(zp)
    assert z.tolist() == [[5, 10]]  # column 0 in the low nibble
    rng = np.random.default_rng(0)
    qq = rng.integers(0, 16, (64, 24))
    assert np.array_equal(awq_ref.wna16_unpack(awq_ref.wna16_pack(qq)), qq)
    zz = rng.integers(0, 16, (4, 24))
    assert np.array_equal(awq_ref.wna16_zeros_unpack(awq_ref.wna16_zeros_pack(zz)), zz)


def test_awq_pack_order_known_answer():
    v = np.arange(8).reshape(1, 8)
    w = awq_ref.awq_pack_cols(v)
    assert int(w.view(np.uint32)[0, 0]) == 0x75316420
    rng = np.random.default_rng(1)
    vv = rng.integers(0, 16, (5, 32))
    assert np.array_equal(awq_ref.awq_unpack_cols(awq_ref.awq_pack_cols(vv)), vv)
    # the sequential (GPTQ) order is a different packing of the same values
    assert not np.array_equal(awq_ref.awq_pack_cols(vv), gptq_ref.pack_cols(vv))


def _scales(rng, shape):
    return rng.uniform(0.002, 0.02, shape).astype(np.float16).astype(np.float32)


def test_wna16_repack_keeps_every_dequantised_weight():
    rng = np.random.default_rng(2)
    K, N, G = 256, 48, 64
    q = rng.integers(0, 16, (K, N))
    z = rng.integers(0, 16, (K // G, N))
    s = _scales(rng, (N, K // G))
    b, zp = awq_ref.wna16_pack(q), awq_ref.wna16_zeros_pack(z)
    want = awq_ref.wna16_dequant_f32(b, zp, s, G)
    # the formula itself: (q - z) * s
    g = np.arange(K) // G
    assert np.array_equal(want, ((q - z[g]) * s.T[g]).astype(np.float32))
    qw, qz, sb = awq_ref.wna16_to_gptq(b, zp, s, G)
    got = gptq_ref.dequant_f32(qw, qz, sb, group_size=G, linear_weight=False)
    assert np.array_equal(got, want)
    # symmetric checkpoints (no zero points) use zero 8
    qw8, qz8, sb8 = awq_ref.wna16_to_gptq(b, None, s, G)
    assert np.all(gptq_ref.unpack_cols(qz8) == 8)
    assert np.array_equal(gptq_ref.dequant_f32(qw8, qz8, sb8, group_size=G, linear_weight=False),
                          awq_ref.wna16_dequant_f32(b, None, s, G))
    # a planted nibble-parity mistake (high nibble = even k) changes the weights
    swapped = ((b >> 4) | (b << 4)).astype(np.uint8)
    assert not np.array_equal(awq_ref.wna16_dequant_f32(swapped, zp, s, G), want)


def test_awq_gemm_repack_keeps_every_dequantised_weight():
    rng = np.random.default_rng(3)
    K, N, G = 256, 64, 128
    q = rng.integers(0, 16, (K, N))
    z = rng.integers(0, 16, (K // G, N))
    s = _scales(rng, (K // G, N)).astype(np.float16).view(np.uint16)
    qw_awq, qz_awq = awq_ref.awq_pack_cols(q), awq_ref.awq_pack_cols(z)
    want = awq_ref.awq_dequant_f32(qw_awq, qz_awq, s, G)
    qw, qz, sb = awq_ref.awq_to_gptq(qw_awq, qz_awq, s)
    assert np.array_equal(gptq_ref.unpack_rows(qw), q)
    assert np.array_equal(gptq_ref.dequant_f32(qw, qz, sb, group_size=G, linear_weight=False), want)
