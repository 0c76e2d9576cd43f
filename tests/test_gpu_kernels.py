"""GPU parity of the individual kernels against the oracle (bit-exact where the path is exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mtp_amd import ops, synth
from oracle import gptq_ref, moe_ref
from tests.helpers import bf16_bits, f16_bits

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)


@pytest.mark.parametrize("E,K,N", [(1, 256, 512), (3, 2048, 512), (2, 512, 2048)])
@pytest.mark.parametrize("linear", [True, False])
def test_dequant_bit_exact(E, K, N, linear):
    _say(f"dequant E={E} K={K} N={N} linear={linear}")
    st = synth.make_projection(E, K, N, synth._gen(77 + K, "cpu"), "cpu")
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        got = ops.dequantize(st.qweight.cuda(), st.qzeros.cuda(), st.scales.cuda(), group_size=128,
                             linear_weight=linear, dtype=dtype).cpu()
        for e in range(E):
            f32 = gptq_ref.dequant_f32(st.qweight[e].numpy(), st.qzeros[e].numpy(),
                                       f16_bits(st.scales[e]), group_size=128, linear_weight=linear)
            want = torch.from_numpy(f32).to(dtype)
            assert torch.equal(got[e].view(torch.uint8), want.contiguous().view(torch.uint8)), (e, dtype)


def test_dequant_reference_kat_and_g_idx():
    _say("dequant KAT")
    int_weight = (np.arange(16 * 8, dtype=np.int32).reshape(16, 8) % 16)
    # pad to the kernel's granularity: K=16 (2 groups of 8), N=8
    zeros = np.stack([np.full(8, 2, np.int32), np.full(8, 5, np.int32)])
    scales = np.stack([np.linspace(0.25, 1.0, 8), np.linspace(1.0, 1.75, 8)]).astype(np.float16)
    g_idx = np.array([0] * 8 + [1] * 8, dtype=np.int32)
    q = torch.from_numpy(gptq_ref.pack_rows(int_weight)).cuda()
    z = torch.from_numpy(gptq_ref.pack_cols(zeros)).cuda()
    s = torch.from_numpy(scales).cuda()
    got = ops.dequantize(q, z, s, torch.from_numpy(g_idx).cuda(), group_size=8,
                         dtype=torch.float32).cpu().numpy()
    expected = ((int_weight - zeros[g_idx]) * scales.astype(np.float32)[g_idx]).T
    assert np.array_equal(got, expected)
    # a permuted g_idx (desc_act-style) follows g_idx, not k // G
    g2 = g_idx[::-1].copy()
    got2 = ops.dequantize(q, z, s, torch.from_numpy(g2).cuda(), group_size=8,
                          dtype=torch.float32).cpu().numpy()
    assert np.array_equal(got2, ((int_weight - zeros[g2]) * scales.astype(np.float32)[g2]).T)


@pytest.mark.parametrize("T,E,H,k,zipf,shared", [(1, 256, 2048, 8, False, False),
                                                 (16, 256, 2048, 8, False, True),
                                                 (64, 256, 2048, 8, True, False),
                                                 (7, 16, 512, 4, False, True),
                                                 (300, 256, 2048, 8, True, True),
                                                 (129, 64, 1536, 8, False, True),
                                                 (1024, 256, 2048, 8, True, False)])
def test_router_bit_exact(T, E, H, k, zipf, shared):
    _say(f"router T={T} E={E} H={H} k={k} zipf={zipf} shared={shared}")
    x = synth.make_tokens(T, H, seed=7 + T)
    rw = synth.make_router(E, H, seed=2000 + T)
    bias = synth.zipf_logit_bias(E, seed=3000 + T) if zipf else None
    sg = synth.make_shared_gate(H, seed=2500) if shared else None
    ids, w, sgate, logits = ops.router_topk(x.cuda(), rw.cuda(), k,
                                            logit_bias=None if bias is None else bias.cuda(),
                                            shared_gate_w=None if sg is None else sg.cuda())
    r_ids, r_w, r_logits = moe_ref.router_topk(bf16_bits(x), bf16_bits(rw), k,
                                               None if bias is None else bias.numpy())
    assert np.array_equal(logits.cpu().numpy(), r_logits), "fp32 logits must be bit-identical"
    assert np.array_equal(ids.cpu().numpy(), r_ids)
    np.testing.assert_allclose(w.cpu().numpy(), r_w, rtol=2e-6, atol=1e-7)
    if shared:
        np.testing.assert_allclose(sgate.cpu().numpy(), moe_ref.shared_gate(bf16_bits(x), bf16_bits(sg)),
                                   rtol=2e-6, atol=1e-7)


def test_router_ties_break_to_lower_id():
    _say("router ties")
    E, H, T = 64, 512, 5
    rw = synth.make_router(E, H, seed=5)
    rw[10] = rw[3]  # identical rows -> identical logits
    rw[40] = rw[3]
    rw[41] = rw[7]
    x = synth.make_tokens(T, H, seed=6)
    ids, _, _, logits = ops.router_topk(x.cuda(), rw.cuda(), 8)
    r_ids, _, r_logits = moe_ref.router_topk(bf16_bits(x), bf16_bits(rw), 8)
    assert np.array_equal(logits.cpu().numpy(), r_logits)
    assert np.array_equal(ids.cpu().numpy(), r_ids)
    zero = torch.zeros(2, H, dtype=torch.bfloat16).cuda()
    ids0, w0, _, _ = ops.router_topk(zero, rw.cuda(), 8)
    assert ids0.cpu().tolist() == [list(range(8))] * 2
    assert torch.allclose(w0.cpu(), torch.full((2, 8), 1 / 8))


@pytest.mark.parametrize("T,k,E,BM,shared,zipf", [(1, 8, 256, 16, False, False),
                                                  (8, 8, 256, 16, True, False),
                                                  (64, 8, 256, 16, False, True),
                                                  (2048, 8, 256, 128, False, True),
                                                  (2048, 8, 256, 128, True, False),
                                                  (33, 4, 16, 128, True, False),
                                                  (1, 3, 8, 4, False, False),
                                                  # block sizes that are not powers of two
                                                  # (the kernels' division fallback)
                                                  (40, 8, 64, 24, False, False),
                                                  (5, 3, 16, 12, True, False),
                                                  (2048, 8, 256, 96, False, True),
                                                  # the two-kernel form from 2 048 slots, and
                                                  # past its 32 768 slots
                                                  (300, 8, 256, 128, True, True),
                                                  (5000, 8, 256, 128, True, True)])
def test_align_bit_exact(T, k, E, BM, shared, zipf):
    _say(f"align T={T} k={k} E={E} BM={BM} shared={shared} zipf={zipf}")
    rng = np.random.default_rng(T + BM)
    if zipf:
        p = np.arange(1, E + 1, dtype=np.float64) ** -1.1
        p /= p.sum()
        ids = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    else:
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    cap = ops.capacity_blocks(T, k, E, shared, BM)
    s, e, n = ops.align(torch.from_numpy(ids).cuda(), E, BM, has_shared=shared)
    rs, re_, rn = moe_ref.align_block_padded(ids, E, BM, has_shared=shared, capacity_blocks=cap)
    assert int(n.item()) == rn
    assert np.array_equal(e.cpu().numpy(), re_)
    assert np.array_equal(s.cpu().numpy(), rs)


def test_align_known_answer():
    _say("align KAT")
    s, e, n = ops.align(torch.tensor([[1, 2, 3]], dtype=torch.int32).cuda(), 8, 4)
    assert int(n.item()) == 12
    assert e.cpu().tolist()[:3] == [1, 2, 3]
    assert s.cpu().tolist()[:12] == [0, 3, 3, 3, 1, 3, 3, 3, 2, 3, 3, 3]


@pytest.mark.parametrize("path", ["decode", "prefill"])
def test_stepwise_entry_points_with_dropped_ids_and_poisoned_ys(path):
    """align -> W1 -> W2 -> moe_sum as separate entry points, with ids outside [0, E) and a ys
    buffer full of NaN: moe_sum skips the dropped slots' rows (W2 never writes them)."""
    from mtp_amd import synth
    from tests.helpers import LAYER_RTOL, experts_to_np, small_layer, to_gpu
    lay = small_layer(6)
    g = to_gpu(lay)
    T, k, E = 12, 4, 16
    rng = np.random.default_rng(60)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    drop = rng.random(ids.shape) < 0.25
    ids[drop] = rng.choice([-3, E, E + 7], size=int(drop.sum()))
    w = rng.uniform(0.1, 0.6, ids.shape).astype(np.float32)
    x = synth.make_tokens(T, 512, seed=61)
    xd, idd, wd = x.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    bm = ops.PREFILL_BLOCK_M if path == "prefill" else ops.DECODE_BLOCK_M
    sorted_ids, eids, ntpp = ops.align(idd, E, bm)
    h = ops.w1_gateup_silu(xd, g.experts, sorted_ids, eids, ntpp, top_k=k, path=path)
    ys = torch.full((T * k, 512), float("nan"), dtype=torch.float32, device="cuda")
    ops.w2_down(h, g.experts, sorted_ids, eids, ntpp, wd.reshape(-1), T=T, top_k=k, path=path, ys=ys)
    out = ops.moe_sum(ys, idd, g.experts)
    torch.cuda.synchronize()
    ref = moe_ref.moe_layer_f32(bf16_bits(x), ids, w, experts_to_np(lay.experts))
    err = moe_ref.rel_err(out.float().cpu().numpy(), ref)
    print(f"  {path}: rel_err={err:.3e}", flush=True)
    assert np.isfinite(err) and err <= LAYER_RTOL


def test_wrappers_refuse_buffers_the_kernels_would_overrun():
    """The tensor wrappers check what the C ABI cannot (it only sees pointers): shapes and
    dtypes of the GPTQ tensors, g_idx's range, align's table sizes and the bias dtype."""
    _say("wrapper argument checks")
    from tests.helpers import small_layer, to_gpu
    st = synth.make_projection(1, 256, 64, synth._gen(5, "cpu"), "cpu")
    q, z, s = st.qweight.cuda(), st.qzeros.cuda(), st.scales.cuda()
    with pytest.raises(ValueError, match="do not match"):
        ops.dequantize(q, z, s[:, :1], group_size=128)
    with pytest.raises(TypeError, match="float16"):
        ops.dequantize(q, z, s.float(), group_size=128)
    bad = torch.zeros(1, 256, dtype=torch.int32, device="cuda")
    bad[0, 7] = 2
    with pytest.raises(ValueError, match="out of range"):
        ops.dequantize(q, z, s, bad, group_size=128)
    g = to_gpu(small_layer(0))
    x = torch.randn(4, 512, device="cuda").to(torch.bfloat16)
    with pytest.raises(ValueError, match="logit_bias"):
        ops.moe_layer(x, g.router_w, g.experts, top_k=4,
                      logit_bias=torch.zeros(16, dtype=torch.bfloat16, device="cuda"))
    ids, w, _, _ = ops.router_topk(x, g.router_w, 4)
    sorted_ids, eids, ntpp = ops.align(ids, 16, 16)
    with pytest.raises(ValueError, match="sorted_ids holds"):
        ops.w1_gateup_silu(x, g.experts, sorted_ids[:16], eids, ntpp, top_k=4, path="decode")


def test_misaligned_workspace_is_refused():
    """Workspace sections are read with 16-byte vector and LDS-direct loads at 256-byte offsets
    from the base: a base off a 256-byte boundary is refused, not run."""
    from tests.helpers import small_layer, to_gpu
    g = to_gpu(small_layer(0))
    x = torch.randn(4, 512, device="cuda").to(torch.bfloat16)
    need = ops.workspace_bytes(4, 4, g.experts, False, "decode")
    ws = torch.zeros(need + 256, dtype=torch.uint8, device="cuda")
    out = ops.moe_layer(x, g.router_w, g.experts, top_k=4, path="decode", workspace=ws[256:])
    with pytest.raises(RuntimeError, match="256-byte aligned"):
        ops.moe_layer(x, g.router_w, g.experts, top_k=4, path="decode", workspace=ws[4:])
    torch.cuda.synchronize()
    want = ops.moe_layer(x, g.router_w, g.experts, top_k=4, path="decode")
    assert torch.equal(out, want)


def test_caller_buffers_off_the_device_or_strided_are_refused():
    """The C ABI sees a caller's workspace and outputs only as pointers and byte counts: a host
    tensor, one on another device or an expanded (stride-0) one is refused by the wrappers, and
    a workspace of another dtype counts its bytes, not its elements."""
    _say("caller buffer checks")
    from tests.helpers import small_layer, to_gpu
    g = to_gpu(small_layer(0))
    x = torch.randn(4, 512, device="cuda").to(torch.bfloat16)
    need = ops.workspace_bytes(4, 4, g.experts, False, "decode")
    want = ops.moe_layer(x, g.router_w, g.experts, top_k=4, path="decode")
    for ws in (torch.empty(need, dtype=torch.uint8),
               torch.empty(1, dtype=torch.uint8, device="cuda").expand(need)):
        with pytest.raises(ValueError, match="workspace must be a contiguous tensor"):
            ops.moe_layer(x, g.router_w, g.experts, top_k=4, path="decode", workspace=ws)
        with pytest.raises(ValueError, match="workspace must be a contiguous tensor"):
            ops.fused_experts(x, torch.zeros(4, 4, dtype=torch.int32, device="cuda"),
                              torch.zeros(4, 4, device="cuda"), g.experts, path="decode",
                              workspace=ws)
    with pytest.raises(ValueError, match="CPU tensor"):
        ops.moe_layer(x, g.router_w, g.experts, top_k=4, path="decode",
                      out=torch.empty(4, 512, dtype=torch.bfloat16))
    norm_w = torch.zeros(512, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="CPU tensor"):
        ops.norm_layer(x, g.router_w, g.experts, norm_w, top_k=4, path="decode",
                       x_out=torch.empty(4, 512, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="CPU tensor"):
        ops.rmsnorm(x.clone(), norm_w, out=torch.empty(4, 512, dtype=torch.bfloat16))
    ids, w, _, _ = ops.router_topk(x, g.router_w, 4)
    sorted_ids, eids, ntpp = ops.align(ids, 16, ops.DECODE_BLOCK_M)
    h = ops.w1_gateup_silu(x, g.experts, sorted_ids, eids, ntpp, top_k=4, path="decode")
    with pytest.raises(ValueError, match="CPU tensor"):
        ops.w2_down(h, g.experts, sorted_ids, eids, ntpp, w.reshape(-1), T=4, top_k=4,
                    path="decode", ys=torch.empty(16, 512, dtype=torch.float32))
    hp = torch.randn(2, 64, device="cuda").to(torch.bfloat16)
    w1 = torch.zeros(1, 32, 64, dtype=torch.bfloat16, device="cuda")
    w2 = torch.zeros(1, 16, 32, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="workspace must be a contiguous tensor"):
        ops.predictor_topk(hp, w1, w2, 4, workspace=torch.empty(1 << 16, dtype=torch.uint8))
    # float32 elements: a quarter of `need` of them covers the workspace
    ws32 = torch.empty((need + 3) // 4, dtype=torch.float32, device="cuda")
    got = ops.moe_layer(x, g.router_w, g.experts, top_k=4, path="decode", workspace=ws32)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
