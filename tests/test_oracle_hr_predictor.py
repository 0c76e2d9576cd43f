"""Pins the oracle's HiddenResidualExpertPredictor forward (oracle/moe_ref.py:hidden_residual_ref).

Reference: training/hidden_residual.py:44-106 (Linear -> SiLU -> LayerNorm encoder, layer and
delta embeddings, SiLU, classifier) and the residual combination of
scripts/train_hidden_residual_predictor_smoke.py:446. Checks: the reference architecture built
from torch's own modules in fp32 on the same (bf16-valued) parameters, closed forms (a zero
classifier gives the bias, a zero LayerNorm weight removes the hidden state, an out-of-range
layer id equals a zero embedding), and the prior + scale * residual combination.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import gptq_ref, moe_ref


def _params(H=256, W=64, L=5, Fw=3, E=40, seed=0):
    g = torch.Generator().manual_seed(seed)
    b = lambda t: gptq_ref.f32_to_bf16_bits(t.numpy().astype(np.float32))  # noqa: E731
    return {
        "enc_w": b((torch.rand(W, H, generator=g) * 2 - 1) / H ** 0.5),
        "enc_b": gptq_ref.bf16_bits_to_f32(b((torch.rand(W, generator=g) * 2 - 1) / H ** 0.5)),
        "ln_w": b(1 + 0.1 * torch.randn(W, generator=g)),
        "ln_b": b(0.1 * torch.randn(W, generator=g)),
        "layer_emb": b(torch.randn(L, W, generator=g)),
        "delta_emb": b(torch.randn(Fw, W, generator=g)),
        "cls_w": b((torch.rand(E, W, generator=g) * 2 - 1) / W ** 0.5),
        "cls_b": gptq_ref.bf16_bits_to_f32(b((torch.rand(E, generator=g) * 2 - 1) / W ** 0.5)),
    }


def _torch_reference(h_bits, p, layer_ids):
    """The reference module's forward in fp32 with torch's own layers."""
    f = gptq_ref.bf16_bits_to_f32
    W, H = p["enc_w"].shape
    enc = torch.nn.Sequential(torch.nn.Linear(H, W), torch.nn.SiLU(), torch.nn.LayerNorm(W))
    with torch.no_grad():
        enc[0].weight.copy_(torch.from_numpy(f(p["enc_w"])))
        enc[0].bias.copy_(torch.from_numpy(p["enc_b"]))
        enc[2].weight.copy_(torch.from_numpy(f(p["ln_w"])))
        enc[2].bias.copy_(torch.from_numpy(f(p["ln_b"])))
        state = enc(torch.from_numpy(f(h_bits)))
        le = torch.from_numpy(f(p["layer_emb"]))[torch.from_numpy(layer_ids).long()]
        de = torch.from_numpy(f(p["delta_emb"]))
        ctx = state[:, None, :] + le[:, None, :] + de[None, :, :]
        return F.linear(F.silu(ctx), torch.from_numpy(f(p["cls_w"])), torch.from_numpy(p["cls_b"])).numpy()


def _hidden(N=6, H=256, seed=1):
    rng = np.random.default_rng(seed)
    return gptq_ref.f32_to_bf16_bits(rng.standard_normal((N, H)).astype(np.float32))


def test_matches_the_reference_architecture_in_fp32():
    p = _params()
    h = _hidden()
    lid = np.array([0, 4, 2, 2, 1, 3], dtype=np.int32)
    _, _, r = moe_ref.hidden_residual_ref(h, p, lid, top_k=5)
    want = _torch_reference(h, p, lid)
    assert r.shape == want.shape == (6, 3, 40)
    # bf16 activations between the layers: agreement to bf16 accuracy
    assert moe_ref.rel_err(r, want) < 2e-2
    # a planted mistake (delta embedding of the wrong row) is far outside that
    p2 = dict(p)
    p2["delta_emb"] = p["delta_emb"][::-1].copy()
    _, _, r2 = moe_ref.hidden_residual_ref(h, p2, lid, top_k=5)
    assert moe_ref.rel_err(r2, want) > 0.1


def test_closed_forms():
    p = _params()
    h = _hidden()
    lid = np.array([0, 1, 2, 3, 4, 0], dtype=np.int32)
    zero = dict(p, cls_w=np.zeros_like(p["cls_w"]))
    _, _, r = moe_ref.hidden_residual_ref(h, zero, lid, top_k=4)
    assert np.array_equal(r, np.broadcast_to(p["cls_b"], r.shape))
    # LayerNorm weight 0: the state is ln_b whatever the hidden state
    flat = dict(p, ln_w=np.zeros_like(p["ln_w"]))
    _, _, ra = moe_ref.hidden_residual_ref(h, flat, lid, top_k=4)
    _, _, rb = moe_ref.hidden_residual_ref(_hidden(seed=9), flat, lid, top_k=4)
    assert np.array_equal(ra, rb)
    # an out-of-range layer id reads a zero embedding
    zl = dict(p, layer_emb=np.concatenate([p["layer_emb"], np.zeros_like(p["layer_emb"][:1])]))
    _, _, rz = moe_ref.hidden_residual_ref(h[:1], zl, np.array([5], np.int32), top_k=4)
    _, _, ro = moe_ref.hidden_residual_ref(h[:1], p, np.array([-3], np.int32), top_k=4)
    assert np.array_equal(rz, ro)


def test_prior_and_scale_combination():
    p = _params()
    h = _hidden()
    lid = np.array([0, 1, 2, 3, 4, 0], dtype=np.int32)
    rng = np.random.default_rng(3)
    prior = rng.standard_normal((6, 3, 40)).astype(np.float32)
    ids, out, r = moe_ref.hidden_residual_ref(h, p, lid, top_k=7, prior=prior, scale=0.5)
    assert np.array_equal(out, (prior + np.float32(0.5) * r).astype(np.float32))
    assert np.array_equal(ids, moe_ref.stable_topk(out.reshape(18, 40), 7).reshape(6, 3, 7))
    per = np.linspace(0.1, 2.0, 6).astype(np.float32)
    _, out2, _ = moe_ref.hidden_residual_ref(h, p, lid, top_k=7, prior=prior, scale_per_example=per)
    assert np.array_equal(out2, (prior + per[:, None, None] * r).astype(np.float32))
