"""GPTQ int4 unpack and dequantisation, restated in numpy.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference: src/mtp_expert_prefetch/repack/gptq_unpack.py
  unpack_cols  :54-68   nibble j of qzeros[g, c] is Z[g, 8c + j]
  unpack_rows  :71-85   nibble j of qweight[r, n] is W[8r + j, n]
  dequantize_gptq_projection :88-131
      W_f32 = (float(W[k, n]) - float(Z[g_idx[k], n])) * float(S[g_idx[k], n])
      transposed to Linear orientation [out, in], then cast (RNE) to bf16.
  synthesize_g_idx :134-148  g_idx[k] = k // group_size
Both packed tensors are read as unsigned 32-bit (``& 0xFFFFFFFF``, :60, :77).
"""

from __future__ import annotations

import numpy as np

PACK = 8  # int4 values per int32


def _as_u32(packed: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(packed).view(np.uint32) if packed.dtype == np.int32 else (
        packed.astype(np.int64) & 0xFFFFFFFF
    ).astype(np.uint32)


def unpack_rows(packed: np.ndarray) -> np.ndarray:
    """[R, C] int32 -> [8R, C] int32 with out[8r + j, c] = nibble j (gptq_unpack.py:71-85)."""
    u = _as_u32(packed)
    rows, cols = u.shape
    out = np.empty((rows * PACK, cols), dtype=np.int32)
    for j in range(PACK):
        out[j::PACK, :] = ((u >> np.uint32(4 * j)) & np.uint32(0xF)).astype(np.int32)
    return out


def unpack_cols(packed: np.ndarray) -> np.ndarray:
    """[R, C] int32 -> [R, 8C] int32 with out[r, 8c + j] = nibble j (gptq_unpack.py:54-68)."""
    u = _as_u32(packed)
    rows, cols = u.shape
    out = np.empty((rows, cols * PACK), dtype=np.int32)
    for j in range(PACK):
        out[:, j::PACK] = ((u >> np.uint32(4 * j)) & np.uint32(0xF)).astype(np.int32)
    return out


def pack_rows(values: np.ndarray) -> np.ndarray:
    """Inverse of unpack_rows (mirrors tests/test_gptq_unpack.py:17-26)."""
    v = (values.astype(np.uint32) & np.uint32(0xF))
    rows, cols = v.shape
    assert rows % PACK == 0
    out = np.zeros((rows // PACK, cols), dtype=np.uint32)
    for j in range(PACK):
        out |= v[j::PACK, :] << np.uint32(4 * j)
    return out.view(np.int32)


def pack_cols(values: np.ndarray) -> np.ndarray:
    """Inverse of unpack_cols (mirrors tests/test_gptq_unpack.py:29-38)."""
    v = (values.astype(np.uint32) & np.uint32(0xF))
    rows, cols = v.shape
    assert cols % PACK == 0
    out = np.zeros((rows, cols // PACK), dtype=np.uint32)
    for j in range(PACK):
        out |= v[:, j::PACK] << np.uint32(4 * j)
    return out.view(np.int32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16, returned as uint16 bit patterns.

    This is the IEEE RNE rule torch uses for ``.to(torch.bfloat16)``; NaNs are
    kept quiet NaNs. Pinned against torch in tests/test_oracle_gptq.py.
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    rounded = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    out = rounded.astype(np.uint16)
    out[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x0040)).astype(np.uint16)
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def synthesize_g_idx(in_features: int, group_size: int = 128) -> np.ndarray:
    """g_idx[k] = k // group_size (gptq_unpack.py:134-148)."""
    return (np.arange(in_features, dtype=np.int32) // np.int32(group_size)).astype(np.int32)


def dequant_f32(qweight: np.ndarray, qzeros: np.ndarray, scales_f16_bits: np.ndarray,
                g_idx: np.ndarray | None = None, *, group_size: int = 128,
                linear_weight: bool = True) -> np.ndarray:
    """fp32 dequantised weight before the final cast (gptq_unpack.py:103-130).

    qweight [K/8, N] int32, qzeros [K/G, N/8] int32, scales [K/G, N] fp16 bits.
    The product (q - z) * s is exact in fp32 (|q - z| <= 15, s an fp16).
    """
    w = unpack_rows(qweight)
    z = unpack_cols(qzeros)
    s = f16_bits_to_f32(scales_f16_bits)
    k_in, n_out = w.shape
    if g_idx is None:
        g_idx = synthesize_g_idx(k_in, group_size)
    g = g_idx.astype(np.int64)
    if g.shape[0] != k_in:
        raise ValueError(f"qweight expands to {k_in} input rows, but g_idx has {g.shape[0]}")
    if z.shape != s.shape or s.shape[1] != n_out:
        raise ValueError("qzeros/scales shape mismatch")
    out = (w.astype(np.float32) - z.astype(np.float32)[g]) * s[g]
    return np.ascontiguousarray(out.T) if linear_weight else out


def dequant_bf16_bits(qweight: np.ndarray, qzeros: np.ndarray, scales_f16_bits: np.ndarray,
                      g_idx: np.ndarray | None = None, *, group_size: int = 128,
                      linear_weight: bool = True) -> np.ndarray:
    """bf16 bit patterns of dequantize_gptq_projection(..., dtype=bf16) (gptq_unpack.py:88-131)."""
    return f32_to_bf16_bits(dequant_f32(qweight, qzeros, scales_f16_bits, g_idx,
                                        group_size=group_size, linear_weight=linear_weight))
