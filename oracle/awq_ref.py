"""AWQ int4 layouts restated on the CPU, and their exact repack into the GPTQ layout.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Layouts (K = in features, N = out features, G = group size, q / z nibbles in [0, 15]):
  wna16   the vLLM fused-MoE int4 layout the reference serves its AWQ checkpoint with, restated
          at tracing/vllm_wna16_group_plan.py:394-470: B uint8 [N, K/2] with q(k, n) in nibble
          k % 2 of byte (n, k // 2) (low nibble = even k); zero points uint8 [N/2, K/G] with
          z(g, n) in nibble n % 2 of byte (n // 2, g); scales [N, K/G]; without zero points the
          zero is 8 (b_zp_num). Dequant: (q - z) * s in fp32, then the compute dtype (:466-469).
  awq     the AutoAWQ GEMM checkpoint layout: qweight int32 [K, N/8] and qzeros int32 [K/G, N/8]
          packed along N in the interleaved order [0, 2, 4, 6, 1, 3, 5, 7] (nibble i of word c holds
          column 8 c + order[i]); scales fp16 [K/G, N].
  gptq    the reference's repacked layout (gptq_unpack.py:54-131): qweight int32 [K/8, N] packed
          along K, qzeros int32 [K/G, N/8] packed along N, both in sequential nibble order.
Every conversion moves nibbles and scale bits only, so the dequantised weights are identical.
"""

from __future__ import annotations

import numpy as np

from oracle import gptq_ref

AWQ_PACK_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


# --------------------------------------------------------------------------- wna16 (vLLM)
def wna16_unpack(b: np.ndarray) -> np.ndarray:
    """uint8 [N, K/2] -> q int32 [K, N]."""
    b = b.astype(np.int64)
    N, K2 = b.shape
    q = np.empty((K2 * 2, N), dtype=np.int32)
    q[0::2, :] = (b & 0xF).T
    q[1::2, :] = (b >> 4).T
    return q


def wna16_pack(q: np.ndarray) -> np.ndarray:
    """q int [K, N] -> uint8 [N, K/2]."""
    q = q.astype(np.int64)
    return np.ascontiguousarray(((q[0::2, :] | (q[1::2, :] << 4)).T).astype(np.uint8))


def wna16_zeros_unpack(zp: np.ndarray) -> np.ndarray:
    """uint8 [N/2, K/G] -> z int32 [K/G, N]."""
    zp = zp.astype(np.int64)
    N2, NG = zp.shape
    z = np.empty((NG, N2 * 2), dtype=np.int32)
    z[:, 0::2] = (zp & 0xF).T
    z[:, 1::2] = (zp >> 4).T
    return z


def wna16_zeros_pack(z: np.ndarray) -> np.ndarray:
    """z int [K/G, N] -> uint8 [N/2, K/G]."""
    z = z.astype(np.int64)
    return np.ascontiguousarray(((z[:, 0::2] | (z[:, 1::2] << 4)).T).astype(np.uint8))


def wna16_dequant_f32(b: np.ndarray, zp: np.ndarray | None, scales_f32: np.ndarray,
                      group_size: int) -> np.ndarray:
    """((q - z) * s) in fp32 as [K, N] (vllm_wna16_group_plan.py:466-469); zp None -> z = 8.
    scales_f32 [N, K/G]."""
    q = wna16_unpack(b)
    K, N = q.shape
    g = np.arange(K) // group_size
    z = np.full((K // group_size, N), 8, np.int32) if zp is None else wna16_zeros_unpack(zp)
    return ((q.astype(np.float32) - z[g].astype(np.float32)) * scales_f32.T[g]).astype(np.float32)


# --------------------------------------------------------------------------- AutoAWQ GEMM
def awq_unpack_cols(packed: np.ndarray) -> np.ndarray:
    """int32 [R, N/8] packed along N in the AWQ order -> int32 [R, N]."""
    u = packed.astype(np.int64) & 0xFFFFFFFF
    R, C = u.shape
    out = np.empty((R, C * 8), dtype=np.int32)
    for i, col in enumerate(AWQ_PACK_ORDER):
        out[:, col::8] = (u >> (4 * i)) & 0xF
    return out


def awq_pack_cols(values: np.ndarray) -> np.ndarray:
    """int [R, N] -> int32 [R, N/8] packed along N in the AWQ order."""
    v = values.astype(np.int64)
    R, N = v.shape
    out = np.zeros((R, N // 8), dtype=np.int64)
    for i, col in enumerate(AWQ_PACK_ORDER):
        out |= v[:, col::8] << (4 * i)
    return (out & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


def awq_dequant_f32(qweight: np.ndarray, qzeros: np.ndarray, scales_f16_bits: np.ndarray,
                    group_size: int) -> np.ndarray:
    """((q - z) * s) in fp32 as [K, N] for the AutoAWQ GEMM layout."""
    q = awq_unpack_cols(qweight)
    z = awq_unpack_cols(qzeros)
    s = gptq_ref.f16_bits_to_f32(scales_f16_bits)
    g = np.arange(q.shape[0]) // group_size
    return ((q.astype(np.float32) - z[g].astype(np.float32)) * s[g]).astype(np.float32)


# --------------------------------------------------------------------------- to GPTQ
def to_gptq(q: np.ndarray, z: np.ndarray, scales_f32: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(q [K, N], z [K/G, N], s [K/G, N] fp16-representable) -> GPTQ (qweight, qzeros, scale
    fp16 bits)."""
    s16 = scales_f32.astype(np.float16)
    assert np.array_equal(s16.astype(np.float32), scales_f32), "scales not exact in fp16"
    return gptq_ref.pack_rows(q), gptq_ref.pack_cols(z), s16.view(np.uint16)


def wna16_to_gptq(b, zp, scales_f32, group_size):
    q = wna16_unpack(b)
    K, N = q.shape
    z = np.full((K // group_size, N), 8, np.int32) if zp is None else wna16_zeros_unpack(zp)
    return to_gptq(q, z, scales_f32.T.copy())


def awq_to_gptq(qweight, qzeros, scales_f16_bits):
    return to_gptq(awq_unpack_cols(qweight), awq_unpack_cols(qzeros),
                   gptq_ref.f16_bits_to_f32(scales_f16_bits))
