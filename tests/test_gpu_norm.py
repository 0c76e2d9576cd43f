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


@pytest.mark.parametrize("T,shared,with_add,in_place,path", [
    (1, False, True, False, "decode"), (2, True, True, False, "decode"),
    (5, False, False, False, "decode"), (16, False, True, False, "decode"),
    (64, True, True, False, "decode"), (7, False, True, True, "decode"),
    (300, False, True, False, "prefill"), (300, True, True, False, "auto")])
def test_norm_layer_equals_norm_then_layer(T, shared, with_add, in_place, path):
    """moe_norm_layer_v1 gives the bits of moe_rmsnorm_v1 followed by moe_layer_v1: on decode
    batches the router normalises its own tokens (same arithmetic as the norm kernel); in place
    (res_out == res_in) and on the prefill path the norm kernel runs first."""
    _say(f"norm layer T={T} shared={shared} add={with_add} in_place={in_place} path={path}")
    layer = to_gpu(synth.make_layer(8, zipf=True, shared=shared))
    g = torch.Generator().manual_seed(T + 101)
    res = torch.randn(T, 2048, generator=g).to(torch.bfloat16).cuda()
    add = (0.5 * torch.randn(T, 2048, generator=g)).to(torch.bfloat16).cuda() if with_add else None
    nw = (0.05 * torch.randn(2048, generator=g)).to(torch.bfloat16).cuda()
    kw = dict(logit_bias=layer.logit_bias, path=path)
    if shared:
        kw.update(shared=layer.shared, shared_gate_w=layer.shared_gate_w)
    # reference: the norm kernel, then the layer
    res_ref = res.clone()
    x_ref = ops.rmsnorm(res_ref, nw, add=add, eps=1e-6)
    y_ref = ops.moe_layer(x_ref, layer.router_w, layer.experts, **kw)
    res_in = res.clone()
    y, res_out, x = ops.norm_layer(res_in, layer.router_w, layer.experts, nw, add=add, eps=1e-6,
                                   res_out=res_in if in_place else None, **kw)
    torch.cuda.synchronize()
    assert torch.equal(x, x_ref)
    assert torch.equal(res_out, res_ref)
    assert torch.equal(y, y_ref)
    if not in_place:
        assert torch.equal(res_in, res)  # the input residual is left as it was


@pytest.mark.parametrize("T,H", [(1, 1024), (6, 1024), (3, 512)])
def test_norm_layer_narrow_hidden(T, H):
    """The router's folded norm over rows shorter than its 2048-column tile (fewer chunks per
    lane) still gives the bits of the norm kernel followed by the layer."""
    _say(f"norm layer narrow hidden T={T} H={H}")
    layer = to_gpu(synth.make_layer(9, num_experts=32, hidden=H, intermediate=512, zipf=True))
    g = torch.Generator().manual_seed(T + 7 * H)
    res = torch.randn(T, H, generator=g).to(torch.bfloat16).cuda()
    add = (0.5 * torch.randn(T, H, generator=g)).to(torch.bfloat16).cuda()
    nw = (0.05 * torch.randn(H, generator=g)).to(torch.bfloat16).cuda()
    res_ref = res.clone()
    x_ref = ops.rmsnorm(res_ref, nw, add=add, eps=1e-6)
    y_ref = ops.moe_layer(x_ref, layer.router_w, layer.experts, top_k=4,
                          logit_bias=layer.logit_bias, path="decode")
    y, res_out, x = ops.norm_layer(res.clone(), layer.router_w, layer.experts, nw, add=add,
                                   eps=1e-6, top_k=4, logit_bias=layer.logit_bias, path="decode")
    torch.cuda.synchronize()
    assert torch.equal(x, x_ref)
    assert torch.equal(res_out, res_ref)
    assert torch.equal(y, y_ref)


def test_norm_layer_chain_equals_unfused_chain():
    """Three chained decode steps (batch 4) through moe_norm_layer_v1 with two alternating
    residual buffers give the bits of the rmsnorm + moe_layer chain."""
    _say("norm layer chain")
    layers = [to_gpu(synth.make_layer(20 + l, zipf=True)) for l in range(3)]
    g = torch.Generator().manual_seed(5)
    res0 = torch.randn(4, 2048, generator=g).to(torch.bfloat16).cuda()
    nws = [(0.05 * torch.randn(2048, generator=g)).to(torch.bfloat16).cuda() for _ in range(3)]
    res_a, y_a = res0.clone(), None
    for ly, nw in zip(layers, nws):
        x = ops.rmsnorm(res_a, nw, add=y_a)
        y_a = ops.moe_layer(x, ly.router_w, ly.experts, logit_bias=ly.logit_bias, path="decode")
    bufs, y_b, cur = [res0.clone(), torch.empty_like(res0)], None, 0
    for ly, nw in zip(layers, nws):
        y_b, _, _ = ops.norm_layer(bufs[cur], ly.router_w, ly.experts, nw, add=y_b,
                                   res_out=bufs[1 - cur], logit_bias=ly.logit_bias, path="decode")
        cur = 1 - cur
    torch.cuda.synchronize()
    assert torch.equal(y_b, y_a)
    assert torch.equal(bufs[cur], res_a)


def test_norm_layer_rejects_partly_overlapping_rows():
    """A residual output that overlaps the input rows at a row offset (not the same rows, which
    is the in-place update) is refused before any launch, as are overlaps of x_out or out with the
    residual rows; the separate rmsnorm refuses overlaps of out, res and add."""
    from mtp_amd._lib import MoeLibraryError
    _say("norm layer partial overlap")
    layer = to_gpu(synth.make_layer(9, num_experts=32, hidden=512, intermediate=512))
    T, H = 4, 512
    buf = torch.randn(2 * T, H).to(torch.bfloat16).cuda()
    nw = torch.zeros(H, dtype=torch.bfloat16, device="cuda")
    res = buf[:T]
    with pytest.raises(MoeLibraryError, match="res_out must equal res_in or not overlap"):
        ops.norm_layer(res, layer.router_w, layer.experts, nw, res_out=buf[1:T + 1], top_k=4,
                       path="decode")
    with pytest.raises(MoeLibraryError, match="must not overlap"):
        ops.norm_layer(res, layer.router_w, layer.experts, nw, x_out=buf[T - 1:2 * T - 1],
                       top_k=4, path="decode")
    with pytest.raises(MoeLibraryError, match="must not overlap"):
        ops.rmsnorm(res, nw, out=buf[2:T + 2])
    torch.cuda.synchronize()
    # disjoint views of the same buffer are fine, and so is the in-place update
    y, r, _ = ops.norm_layer(buf[:T], layer.router_w, layer.experts, nw, res_out=buf[T:],
                             top_k=4, path="decode")
    y2, r2, _ = ops.norm_layer(buf[T:].clone(), layer.router_w, layer.experts, nw, top_k=4,
                               path="decode")
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
