"""GPU parity of the decoder-step residual add + RMSNorm (moe_rmsnorm_v1) and of MoE layers
chained through it (the decode-step caller of the layer).

Tolerances: the residual sum is bit-exact (one fp32 add, one bf16 rounding); the normalised
output is within one bf16 ulp of the oracle (the fp32 sum of squares runs in the kernel's own
fixed order); chained layers meet the layer tolerance LAYER_RTOL at every step, each step
checked against the oracle fed that step's actual input.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mtp_amd import ops, synth
from oracle import gptq_ref, moe_ref
from tests.helpers import LAYER_RTOL, bf16_bits, experts_to_np, small_layer, to_gpu

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _within_one_ulp(got_bits: np.ndarray, want_bits: np.ndarray) -> None:
    g = gptq_ref.bf16_bits_to_f32(got_bits).astype(np.float64)
    w = gptq_ref.bf16_bits_to_f32(want_bits).astype(np.float64)
    assert np.all(np.abs(g - w) <= np.abs(w) * 2.0 ** -7 + 1e-30)
    assert np.mean(got_bits == want_bits) > 0.99


@pytest.mark.parametrize("T,H,with_add", [(7, 512, False), (5, 2048, True), (3, 2560, True),
                                          (64, 2048, True)])
def test_rmsnorm_matches_oracle(T, H, with_add):
    _say(f"rmsnorm T={T} H={H} add={with_add}")
    g = torch.Generator().manual_seed(T * 31 + H)
    res = torch.randn(T, H, generator=g).to(torch.bfloat16)
    add = (0.5 * torch.randn(T, H, generator=g)).to(torch.bfloat16) if with_add else None
    w = (0.05 * torch.randn(H, generator=g)).to(torch.bfloat16)
    want_res, want_out = moe_ref.rmsnorm_ref(_bits(res), _bits(w),
                                             add_bits=_bits(add) if with_add else None, eps=1e-6)
    res_g = res.cuda()
    out = ops.rmsnorm(res_g, w.cuda(), add=add.cuda() if with_add else None, eps=1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(res_g), want_res)
    _within_one_ulp(_bits(out), want_out)


def test_rmsnorm_rejects_bad_shapes():
    x = torch.zeros(2, 12, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(Exception):
        ops.rmsnorm(x, torch.zeros(12, dtype=torch.bfloat16, device="cuda"))  # hidden % 8 != 0


def test_decode_chain_through_norm():
    """Three MoE layers in a decode loop: h_l = rmsnorm(res), y_l = layer_l(h_l), res += y_l."""
    T, k, L, H = 4, 4, 3, 512
    _say(f"decode chain T={T} layers={L}")
    layers_cpu = [small_layer(10 + l) for l in range(L)]
    layers = [to_gpu(ly) for ly in layers_cpu]
    g = torch.Generator().manual_seed(11)
    norm_w = [(0.05 * torch.randn(H, generator=g)).to(torch.bfloat16) for _ in range(L + 1)]
    res = synth.make_tokens(T, H, seed=21).cuda()
    h = ops.rmsnorm(res, norm_w[0].cuda())
    for l in range(L):
        h_bits = _bits(h)
        y, ids, _ = ops.moe_layer(h, layers[l].router_w, layers[l].experts, top_k=k, path="decode",
                                  return_routing=True)
        torch.cuda.synchronize()
        ref, r_ids, _, _ = moe_ref.moe_layer_ref(h_bits, bf16_bits(layers_cpu[l].router_w),
                                                 experts_to_np(layers_cpu[l].experts), top_k=k)
        assert np.array_equal(ids.cpu().numpy(), r_ids), f"layer {l}: routing ids"
        err = moe_ref.rel_err(y.float().cpu().numpy(), ref)
        _say(f"  layer {l}: rel_err={err:.3e}")
        assert err <= LAYER_RTOL
        res_bits = _bits(res)
        h = ops.rmsnorm(res, norm_w[l + 1].cuda(), add=y)
        torch.cuda.synchronize()
        want_res, want_h = moe_ref.rmsnorm_ref(res_bits, _bits(norm_w[l + 1]), add_bits=_bits(y))
        assert np.array_equal(_bits(res), want_res)
        _within_one_ulp(_bits(h), want_h)
