"""The decoder-step RMSNorm oracle (mtp_rms_norm, mtp/extra_tensors.py:40-48) pinned by closed
forms and a float64 evaluation, independent of the oracle's own float32 formula."""

from __future__ import annotations

import numpy as np
import torch

from oracle import gptq_ref, moe_ref


def _bits(x: np.ndarray) -> np.ndarray:
    return gptq_ref.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def _f(bits: np.ndarray) -> np.ndarray:
    return gptq_ref.bf16_bits_to_f32(bits)


def test_constant_row_closed_form():
    """A row of the constant c normalises to c / sqrt(c^2 + eps), times (1 + w)."""
    H, eps = 64, 1e-6
    res = _bits(np.full((3, H), [[0.5], [-2.0], [3.0]], dtype=np.float32))
    w = _bits(np.linspace(-0.5, 0.5, H))
    _, out = moe_ref.rmsnorm_ref(res, w, eps=eps)
    for t, c in enumerate((0.5, -2.0, 3.0)):
        want = _bits(np.float32(c / np.sqrt(c * c + eps)) * (1.0 + _f(w)))
        assert np.array_equal(out[t], want)


def test_one_hot_row_and_zero_weight():
    """A one-hot row of value a has mean a^2 / H, so the hot element becomes sqrt(H) (w = 0)."""
    H = 256
    x = np.zeros((1, H), dtype=np.float32)
    x[0, 17] = 4.0
    _, out = moe_ref.rmsnorm_ref(_bits(x), _bits(np.zeros(H)), eps=0.0)
    o = _f(out)
    assert o[0, 17] == np.float32(16.0) and np.count_nonzero(o) == 1


def test_float64_agreement_and_residual_add():
    """Random rows against a float64 evaluation: within one bf16 ulp; the residual sum is the
    bf16 rounding of the fp32 sum (torch's bf16 cast as the independent rounding)."""
    g = torch.Generator().manual_seed(3)
    T, H = 16, 2048
    a = torch.randn(T, H, generator=g).to(torch.bfloat16)
    b = (0.3 * torch.randn(T, H, generator=g)).to(torch.bfloat16)
    w = (0.05 * torch.randn(H, generator=g)).to(torch.bfloat16)
    res_bits = a.view(torch.int16).numpy().view(np.uint16)
    add_bits = b.view(torch.int16).numpy().view(np.uint16)
    w_bits = w.view(torch.int16).numpy().view(np.uint16)
    new_res, out = moe_ref.rmsnorm_ref(res_bits, w_bits, add_bits=add_bits, eps=1e-6)
    want_res = (a.float() + b.float()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(new_res, want_res)
    x = _f(new_res).astype(np.float64)
    ref = x / np.sqrt((x ** 2).mean(-1, keepdims=True) + 1e-6) * (1.0 + _f(w_bits).astype(np.float64))
    got = _f(out).astype(np.float64)
    ulp = np.abs(ref) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - ref) <= ulp)


def test_scale_invariance():
    """RMSNorm is invariant to scaling the row by a power of two (exact in bf16)."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, 512, generator=g).to(torch.bfloat16)
    w = (0.1 * torch.randn(512, generator=g)).to(torch.bfloat16)
    wb = w.view(torch.int16).numpy().view(np.uint16)
    _, o1 = moe_ref.rmsnorm_ref(x.view(torch.int16).numpy().view(np.uint16), wb, eps=0.0)
    _, o2 = moe_ref.rmsnorm_ref((8 * x).view(torch.int16).numpy().view(np.uint16), wb, eps=0.0)
    assert np.array_equal(o1, o2)
