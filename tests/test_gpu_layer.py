"""GPU parity of the fused W4A16 MoE layer against the fp32-accumulated oracle.

Routing ids must be bit-exact; layer outputs within LAYER_RTOL (1e-2) normwise relative error
max|out - ref| / max|ref| (bf16 output against an fp32-accumulated reference that uses the
reference's bit-exact bf16 dequantised weights).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mtp_amd import ops, synth
from mtp_amd.moe import MoeBlock
from oracle import moe_ref
from tests.helpers import LAYER_RTOL, bf16_bits, experts_to_np, small_layer, to_gpu

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)


def _check_layer(layer_cpu, T, top_k, path, seed=7):
    x = synth.make_tokens(T, layer_cpu.experts.hidden_size, seed=seed)
    g = to_gpu(layer_cpu)
    out, ids, w = ops.moe_layer(x.cuda(), g.router_w, g.experts, top_k=top_k,
                                logit_bias=g.logit_bias, shared=g.shared,
                                shared_gate_w=g.shared_gate_w, path=path, return_routing=True)
    torch.cuda.synchronize()
    ref, r_ids, r_w, _ = moe_ref.moe_layer_ref(
        bf16_bits(x), bf16_bits(layer_cpu.router_w), experts_to_np(layer_cpu.experts), top_k=top_k,
        logit_bias=None if layer_cpu.logit_bias is None else layer_cpu.logit_bias.numpy(),
        shared=None if layer_cpu.shared is None else experts_to_np(layer_cpu.shared),
        shared_gate_w_bits=None if layer_cpu.shared_gate_w is None else bf16_bits(layer_cpu.shared_gate_w))
    assert np.array_equal(ids.cpu().numpy(), r_ids), "routing ids must be bit-exact"
    np.testing.assert_allclose(w.cpu().numpy(), r_w, rtol=2e-6, atol=1e-7)
    err = moe_ref.rel_err(out.float().cpu().numpy(), ref)
    _say(f"  rel_err={err:.3e}")
    assert err <= LAYER_RTOL
    return out


@pytest.mark.parametrize("T", [1, 3, 16, 40])
@pytest.mark.parametrize("path", ["decode", "prefill"])
def test_small_layer(T, path):
    _say(f"small layer T={T} path={path}")
    _check_layer(small_layer(0), T, 4, path)


@pytest.mark.parametrize("T", [4, 8])
def test_token_sum_w2_with_shared_expert(T):
    """Up to 8 tokens W2 is token-major and sums each token's weighted rows itself (one wave per
    routed slot plus one for the gated shared expert)."""
    _say(f"token-sum W2 with shared expert T={T}")
    _check_layer(small_layer(2, shared=True), T, 4, "decode")


@pytest.mark.parametrize("T,path", [(16, "decode"), (16, "prefill"), (1, "decode"), (32, "decode"),
                                    (64, "decode"), (256, "auto"), (320, "auto")])
def test_config1_full_shape(T, path):
    """Config 1: hidden 2048, 256 experts, intermediate 512, top-8, 16 tokens; and batches on
    either side of the auto path switch (2 048 slots: decode, 2 560: prefill)."""
    _say(f"config1 T={T} path={path}")
    _check_layer(synth.make_layer(0), T, 8, path)


@pytest.mark.parametrize("E,H,I,G,T,shared", [(32, 1024, 1024, 64, 200, True),
                                               (16, 1536, 512, 256, 130, False),
                                               (24, 512, 256, 128, 300, True),
                                               (24, 512, 256, 128, 1100, True)])
def test_prefill_shapes_and_groups(E, H, I, G, T, shared):
    """Prefill GEMMs over other hidden / intermediate sizes, group sizes 64 and 256, with and
    without the shared expert (its block reads the shared projections). T = 1100 (5500 slots)
    takes the large-input align, which also orders the blocks heaviest first for the GEMMs."""
    _say(f"prefill shape E={E} H={H} I={I} G={G} T={T} shared={shared}")
    layer = synth.make_layer(3, num_experts=E, hidden=H, intermediate=I, zipf=True, shared=shared,
                             group=G)
    _check_layer(layer, T, 4, "prefill")


@pytest.mark.parametrize("E,H,I,G,shared", [(32, 1024, 512, 128, False), (24, 1024, 256, 64, True),
                                             (20, 1536, 1024, 256, False)])
@pytest.mark.parametrize("T", [1, 2, 5, 40])
def test_decode_shapes_and_groups(E, H, I, G, shared, T):
    """Decode path over other hidden / intermediate / group sizes: hidden 1024 gives the fused
    W1 + W2 slot grid four waves over K (hidden / 256); groups 64 and 256 and hidden 1536 take
    the unfused slot grid; 5 and 40 tokens the blocked kernels and the token-sum W2."""
    _say(f"decode shape E={E} H={H} I={I} G={G} shared={shared} T={T}")
    layer = synth.make_layer(4, num_experts=E, hidden=H, intermediate=I, zipf=True, shared=shared,
                             group=G)
    _check_layer(layer, T, 4, "decode")


@pytest.mark.parametrize("T", [1, 32])
def test_config4_shared_expert(T):
    """Config 4: routed top-8 plus a sigmoid-gated int4 shared expert."""
    _say(f"config4 T={T}")
    _check_layer(synth.make_layer(1, shared=True), T, 8, "auto")


def test_decode_and_prefill_paths_agree_on_zipf_batch():
    _say("decode vs prefill T=64 zipf")
    layer = to_gpu(synth.make_layer(2, zipf=True))
    x = synth.make_tokens(64, seed=11).cuda()
    outs = [ops.moe_layer(x, layer.router_w, layer.experts, logit_bias=layer.logit_bias, path=p)
            for p in ("decode", "prefill")]
    for o in outs[1:]:
        assert moe_ref.rel_err(o.float().cpu().numpy(), outs[0].float().cpu().numpy()) < 1e-2


def test_fused_experts_and_moe_tokens_api():
    _say("moe_tokens API")
    layer = small_layer(3, shared=True)
    g = to_gpu(layer)
    T, k = 6, 4
    x = synth.make_tokens(T, 512, seed=3)
    rng = np.random.default_rng(0)
    ids = np.stack([rng.choice(16, k, replace=False) for _ in range(T)]).astype(np.int32)
    ids[0, 1] = ids[0, 0]  # a duplicated expert in one token is summed twice
    w = rng.uniform(0.05, 0.5, (T, k)).astype(np.float32)
    block = MoeBlock(g.experts, g.router_w, shared_expert=g.shared,
                     shared_expert_gate_weight=g.shared_gate_w, top_k=k)
    out = block.moe_tokens(x.cuda().view(2, 3, 512), torch.from_numpy(ids).view(2, 3, k),
                           torch.from_numpy(w).view(2, 3, k))
    sg = moe_ref.shared_gate(bf16_bits(x), bf16_bits(layer.shared_gate_w))
    ref = moe_ref.moe_layer_f32(bf16_bits(x), ids, w, experts_to_np(layer.experts),
                                shared=experts_to_np(layer.shared), shared_gate_values=sg)
    assert moe_ref.rel_err(out.view(T, 512).float().cpu().numpy(), ref) <= LAYER_RTOL
    with pytest.raises(KeyError):
        block.moe_tokens(x.cuda().view(2, 3, 512), torch.full((2, 3, k), 99), torch.from_numpy(w).view(2, 3, k))


def test_empty_batch_gives_empty_outputs():
    """A batch of no tokens is a no-op of every layer entry point (T = 0 returns at once; align
    writes only ntpp = 0 and takes NULL tables); the shapes come back empty."""
    _say("empty batch")
    g = to_gpu(small_layer(3, shared=True))
    sh = dict(shared=g.shared, shared_gate_w=g.shared_gate_w)
    x = torch.empty(0, 512, dtype=torch.bfloat16, device="cuda")
    for path in ("auto", "decode", "prefill"):
        out, ids, w = ops.moe_layer(x, g.router_w, g.experts, top_k=4, path=path,
                                    return_routing=True, **sh)
        assert out.shape == (0, 512) and ids.shape == (0, 4) and w.shape == (0, 4)
    r_ids, r_w, gate, logits = ops.router_topk(x, g.router_w, 4, shared_gate_w=g.shared_gate_w)
    assert r_ids.shape == (0, 4) and r_w.shape == (0, 4) and gate.shape == (0,)
    assert logits.shape == (0, 16)
    sorted_ids, eids, ntpp = ops.align(r_ids, 16, ops.DECODE_BLOCK_M, has_shared=True)
    assert sorted_ids.numel() == 0 and eids.numel() == 0
    h = ops.w1_gateup_silu(x, g.experts, sorted_ids, eids, ntpp, top_k=4, shared=g.shared,
                           path="decode")
    ys = ops.w2_down(h, g.experts, sorted_ids, eids, ntpp, r_w.reshape(-1), T=0, top_k=4,
                     shared=g.shared, path="decode")
    assert h.shape == (0, 256) and ys.shape == (0, 512)
    assert ops.moe_sum(ys, r_ids, g.experts, has_shared=True).shape == (0, 512)
    assert ops.fused_experts(x, r_ids, r_w, g.experts, **sh).shape == (0, 512)
    norm_w = torch.zeros(512, dtype=torch.bfloat16, device="cuda")
    out, res_out, xn = ops.norm_layer(x, g.router_w, g.experts, norm_w, top_k=4, **sh)
    assert out.shape == res_out.shape == xn.shape == (0, 512)
    block = MoeBlock(g.experts, g.router_w, shared_expert=g.shared,
                     shared_expert_gate_weight=g.shared_gate_w, top_k=4)
    assert block(x.view(2, 0, 512)).shape == (2, 0, 512)
    assert block.moe_tokens(x.view(2, 0, 512), torch.empty(2, 0, 4, dtype=torch.long),
                            torch.empty(2, 0, 4)).shape == (2, 0, 512)
    torch.cuda.synchronize()
    assert int(ntpp.item()) == 0


def test_expert_row_indirection_matches_direct():
    """A slot pool: experts held in arbitrary rows, addressed through expert_row."""
    _say("expert_row indirection")
    layer = to_gpu(small_layer(4))
    E = 16
    perm = torch.randperm(E, generator=torch.Generator().manual_seed(1))
    from mtp_amd.weights import GptqStack, MoeExperts
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(E)

    def permute(st: GptqStack) -> GptqStack:
        return GptqStack(st.qweight[perm.cuda()].contiguous(), st.qzeros[perm.cuda()].contiguous(),
                         st.scales[perm.cuda()].contiguous())
    pooled = MoeExperts(permute(layer.experts.gate), permute(layer.experts.up),
                        permute(layer.experts.down), 128,
                        expert_row=inv.to(torch.int32).cuda(), num_experts=E)
    for T in (6, 9):  # 6: W2 sums the token's rows itself; 9: blocked W2 + moe_sum
        x = synth.make_tokens(T, 512, seed=4).cuda()
        for path in ("decode", "prefill"):
            a = ops.moe_layer(x, layer.router_w, layer.experts, top_k=4, path=path)
            b = ops.moe_layer(x, layer.router_w, pooled, top_k=4, path=path)
            assert torch.equal(a, b)


def test_workspace_reusable_across_sizes_and_paths():
    """One workspace reused by calls of different T and path gives the fresh-workspace result."""
    _say("workspace reuse")
    layer = to_gpu(synth.make_layer(6, zipf=True))
    ws = torch.full((ops.workspace_bytes(2048, 8, layer.experts, False, "prefill") + 4096,), 0x5A,
                    dtype=torch.uint8, device="cuda")
    results = {}
    for T, path in ((1, "decode"), (64, "decode"), (2048, "prefill"), (64, "decode"), (1, "decode"),
                    (2048, "prefill"), (65, "decode")):
        x = synth.make_tokens(T, seed=T).cuda()
        out = ops.moe_layer(x, layer.router_w, layer.experts, logit_bias=layer.logit_bias,
                            path=path, workspace=ws)
        torch.cuda.synchronize()
        if (T, path) in results:
            assert torch.equal(results[(T, path)], out), (T, path)
        else:
            fresh = ops.moe_layer(x, layer.router_w, layer.experts, logit_bias=layer.logit_bias,
                                  path=path)
            assert torch.equal(fresh, out), (T, path)
        results[(T, path)] = out


def test_layer_is_deterministic():
    _say("determinism")
    layer = to_gpu(synth.make_layer(5, zipf=True))
    x = synth.make_tokens(32, seed=5).cuda()
    outs = [ops.moe_layer(x, layer.router_w, layer.experts, logit_bias=layer.logit_bias) for _ in range(3)]
    assert all(torch.equal(outs[0], o) for o in outs[1:])


@pytest.mark.parametrize("path,T", [("decode", 1), ("decode", 2), ("decode", 5), ("prefill", 64),
                                    ("decode", 64)])
def test_dropped_slots_contribute_zero(path, T):
    """Ids outside [0, E) are dropped (reference: vllm_router_trace.py:14138-14153); the other
    slots of the token still count, on every path including the fused W2 + sum."""
    _say(f"dropped slots path={path} T={T}")
    lay = small_layer(4)
    g = to_gpu(lay)
    rng = np.random.default_rng(40 + T)
    ids = np.stack([rng.choice(16, size=4, replace=False) for _ in range(T)]).astype(np.int32)
    drop = rng.random(ids.shape) < 0.3
    ids[drop] = rng.choice([-1, 16, 40], size=int(drop.sum()))
    w = rng.uniform(0.1, 1.0, size=ids.shape).astype(np.float32)
    x = synth.make_tokens(T, 512, seed=41 + T)
    got = ops.fused_experts(x.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(),
                            g.experts, path=path)
    torch.cuda.synchronize()
    ref = moe_ref.moe_layer_f32(bf16_bits(x), ids, w, experts_to_np(lay.experts))
    err = moe_ref.rel_err(got.float().cpu().numpy(), ref)
    _say(f"  rel_err={err:.3e}")
    assert np.isfinite(err) and err <= LAYER_RTOL


@pytest.mark.parametrize("case", ["one_expert", "mixed"])
def test_decode_repeated_ids(case):
    """Caller-given ids may repeat an expert within and across tokens: at decode size the kernels
    group slots per expert themselves (16 per workgroup), here with up to 64 slots of one expert."""
    _say(f"repeated ids case={case}")
    lay = small_layer(5)
    g = to_gpu(lay)
    T, k = 8, 8
    rng = np.random.default_rng(55)
    if case == "one_expert":
        ids = np.full((T, k), 3, dtype=np.int32)
    else:
        ids = rng.choice([1, 2, 3, 9], size=(T, k)).astype(np.int32)
    w = rng.uniform(0.05, 0.3, size=(T, k)).astype(np.float32)
    x = synth.make_tokens(T, 512, seed=56)
    ref = moe_ref.moe_layer_f32(bf16_bits(x), ids, w, experts_to_np(lay.experts))
    for path in ("decode", "prefill"):
        got = ops.fused_experts(x.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(),
                                g.experts, path=path)
        torch.cuda.synchronize()
        err = moe_ref.rel_err(got.float().cpu().numpy(), ref)
        _say(f"  {path}: rel_err={err:.3e}")
        assert np.isfinite(err) and err <= LAYER_RTOL


def _workspace_offsets(T, k, E, has_shared, bm, cap):
    """Byte offsets of the routing sections of a layer workspace, in the library's order
    (logits, router-row norms, ids, weights, sorted slot ids, block experts, ntpp, block order;
    each 256-byte aligned)."""
    def a256(n):
        return (n + 255) // 256 * 256
    slots = T * k + (T if has_shared else 0)
    sizes = (("logits", T * (E + 1) * 4), ("norms", (E + 1) * 4), ("ids", T * k * 4), ("w", slots * 4),
             ("sorted", cap * bm * 4), ("eids", cap * 4), ("ntpp", 256), ("border", cap * 4))
    off, out = 0, {}
    for name, n in sizes:
        out[name] = off
        off += a256(n)
    return out


@pytest.mark.parametrize("shared", [False, True])
def test_fused_prefill_align_layout(shared):
    """The fused layer's large-input align (per-chunk ranks, then one workgroup per chunk that
    derives the group offsets and scatters its own slots) writes the oracle's stable layout, the
    unused tail, and the block order heaviest first (16-row subtiles holding slots, ties in
    block order)."""
    T, k, E, BM = 2048, 8, 256, ops.PREFILL_BLOCK_M
    _say(f"fused prefill align layout T={T} shared={shared}")
    layer = to_gpu(synth.make_layer(5, num_experts=E, hidden=512, intermediate=256, zipf=True,
                                    shared=shared))
    x = synth.make_tokens(T, 512, seed=13).cuda()
    need = ops.workspace_bytes(T, k, layer.experts, shared, "prefill")
    ws = torch.full((need,), 0x5A, dtype=torch.uint8, device="cuda")
    _, ids, _ = ops.moe_layer(x, layer.router_w, layer.experts, top_k=k,
                              logit_bias=layer.logit_bias, shared=layer.shared,
                              shared_gate_w=layer.shared_gate_w, path="prefill", workspace=ws,
                              return_routing=True)
    torch.cuda.synchronize()
    cap = ops.capacity_blocks(T, k, E, shared, BM)
    o = _workspace_offsets(T, k, E, shared, BM, cap)
    i32 = ws.view(torch.int32).cpu().numpy()
    got_sorted = i32[o["sorted"] // 4: o["sorted"] // 4 + cap * BM]
    got_eids = i32[o["eids"] // 4: o["eids"] // 4 + cap]
    got_ntpp = int(i32[o["ntpp"] // 4])
    rs, re_, rn = moe_ref.align_block_padded(ids.cpu().numpy(), E, BM, has_shared=shared,
                                             capacity_blocks=cap)
    assert got_ntpp == rn
    assert np.array_equal(got_sorted, rs)
    assert np.array_equal(got_eids, re_)
    n_slots = T * k + (T if shared else 0)
    nblk = rn // BM
    cls = [(int((rs[b * BM:(b + 1) * BM] < n_slots).sum()) + 15) // 16 for b in range(nblk)]
    want = sorted(range(nblk), key=lambda b: (-cls[b], b))
    got_border = i32[o["border"] // 4: o["border"] // 4 + nblk]
    assert list(got_border) == want


@pytest.mark.parametrize("T", [8, 64])
def test_config2_zipf_decode_full_shape(T):
    """Config 2 at full shape with the Zipf(1.1) routing skew, decode path, against the oracle
    (ids bit-exact, weights, layer output)."""
    _say(f"config2 zipf decode T={T}")
    _check_layer(synth.make_layer(T % 40, zipf=True), T, 8, "decode", seed=100 + T)


def _hottest_last_block_tokens(ids: np.ndarray, block_m: int) -> tuple[int, np.ndarray]:
    """Tokens of the hottest expert's last align block (slots sorted by flat id within the
    expert's group, so the last block holds its highest flat ids)."""
    flat = ids.reshape(-1)
    counts = np.bincount(flat, minlength=int(flat.max()) + 1)
    hot = int(np.argmax(counts))
    slots = np.nonzero(flat == hot)[0]
    c = len(slots)
    start = (-(-c // block_m) - 1) * block_m
    return hot, np.unique(slots[start:] // ids.shape[1])


def test_config3_prefill_full_shape_zipf():
    """Config 3: 2048 tokens through one full-shape layer with Zipf(1.1) skew on the prefill
    path. Every token's ids are compared bit-exact; the output is compared against the oracle
    on a token subsample that holds every token of the hottest expert's last align block, a
    stride-16 sample and the last token."""
    T, k = 2048, 8
    _say(f"config3 prefill T={T}")
    layer_cpu = synth.make_layer(3, zipf=True)
    g = to_gpu(layer_cpu)
    x = synth.make_tokens(T, seed=7)
    out, ids, w = ops.moe_layer(x.cuda(), g.router_w, g.experts, top_k=k,
                                logit_bias=g.logit_bias, path="prefill", return_routing=True)
    torch.cuda.synchronize()
    x_bits = bf16_bits(x)
    r_ids, r_w, _ = moe_ref.router_topk(x_bits, bf16_bits(layer_cpu.router_w), k,
                                        layer_cpu.logit_bias.numpy())
    assert np.array_equal(ids.cpu().numpy(), r_ids), "routing ids must be bit-exact"
    np.testing.assert_allclose(w.cpu().numpy(), r_w, rtol=2e-6, atol=1e-7)
    counts = np.bincount(r_ids.reshape(-1), minlength=256)
    hot, hot_tokens = _hottest_last_block_tokens(r_ids, ops.PREFILL_BLOCK_M)
    _say(f"  hottest expert {hot}: {counts[hot]} slots "
         f"({-(-counts[hot] // ops.PREFILL_BLOCK_M)} blocks), last block {len(hot_tokens)} tokens")
    assert counts[hot] > 8 * ops.PREFILL_BLOCK_M  # the skew spreads the expert over many blocks
    sub = np.unique(np.concatenate([hot_tokens, np.arange(0, T, 16), [T - 1]]))
    ref = moe_ref.moe_layer_f32(x_bits[sub], r_ids[sub], r_w[sub], experts_to_np(layer_cpu.experts))
    err = moe_ref.rel_err(out.float().cpu().numpy()[sub], ref)
    _say(f"  {len(sub)} tokens checked, rel_err={err:.3e}")
    assert err <= LAYER_RTOL


@pytest.mark.parametrize("shared", [False, True])
def test_prefill_router_certificate_on_ties(shared):
    """The prefill router selects on approximate MFMA logits and recomputes canonical logits for
    the candidates its error bound cannot separate. Router rows that are exactly equal (ties:
    the lower id first) or one bf16 ulp apart (near-ties inside the bound) force that path; ids
    and weights must still equal the oracle's canonical ones for every token."""
    T, k, E, H = 384, 8, 64, 1024
    _say(f"prefill router certificate on ties T={T} shared={shared}")
    layer = synth.make_layer(7, num_experts=E, hidden=H, intermediate=256, shared=shared)
    rw = layer.router_w.float().clone()
    g = torch.Generator().manual_seed(77)
    v = torch.randn(H, generator=g) * 0.05
    for e in (3, 9, 10, 40):          # exact ties
        rw[e] = v
    near = v.to(torch.bfloat16).float().clone()
    near[17] = torch.nextafter(near[17].to(torch.bfloat16), torch.tensor(1e9).to(torch.bfloat16)).float()
    rw[11] = near                      # one ulp away in one element
    rw[41] = -v                        # the opposite direction: never selected with the others
    layer.router_w = rw.to(torch.bfloat16)
    gl = to_gpu(layer)
    x = synth.make_tokens(T, H, seed=78)
    out, ids, w = ops.moe_layer(x.cuda(), gl.router_w, gl.experts, top_k=k, shared=gl.shared,
                                shared_gate_w=gl.shared_gate_w, path="prefill",
                                return_routing=True)
    torch.cuda.synchronize()
    r_ids, r_w, r_logits = moe_ref.router_topk(bf16_bits(x), bf16_bits(layer.router_w), k)
    tied = np.isin(r_ids, [3, 9, 10, 11, 40]).sum(axis=1)
    _say(f"  tokens with >= 2 tied experts in the top-{k}: {int((tied >= 2).sum())}")
    assert (tied >= 2).sum() > T // 4
    assert np.array_equal(ids.cpu().numpy(), r_ids), "routing ids must be bit-exact"
    np.testing.assert_allclose(w.cpu().numpy(), r_w, rtol=2e-6, atol=1e-7)
    if shared:
        sg = moe_ref.shared_gate(bf16_bits(x), bf16_bits(layer.shared_gate_w))
        ref = moe_ref.moe_layer_f32(bf16_bits(x), r_ids, r_w, experts_to_np(layer.experts),
                                    shared=experts_to_np(layer.shared), shared_gate_values=sg)
        assert moe_ref.rel_err(out.float().cpu().numpy(), ref) <= LAYER_RTOL


@pytest.mark.parametrize("T,path,top_k", [(3, "decode", 8), (3, "decode", 16), (40, "decode", 8),
                                          (9, "decode", 16), (300, "prefill", 8),
                                          (1100, "prefill", 8)])
def test_max_expert_count_with_shared_expert(T, path, top_k):
    """The largest supported expert set: 512 routed experts plus the shared one (513 groups in
    align, 513 logits per token in the routers); top-16 in the decode routing, and the
    large-input align's chunk count at 513 groups for 1100 tokens."""
    _say(f"512 experts + shared T={T} path={path} top_k={top_k}")
    layer = synth.make_layer(5, num_experts=512, hidden=512, intermediate=256, zipf=True,
                             shared=True)
    _check_layer(layer, T, top_k, path)


@pytest.mark.parametrize("T,path,top_k", [(1, "decode", 1), (7, "decode", 1), (64, "decode", 2),
                                          (300, "prefill", 1), (2600, "auto", 1),
                                          (700, "auto", 2)])
def test_one_and_two_experts_per_token(T, path, top_k):
    """top_k 1 and 2 (the renormalised weight of a single expert is exactly 1): every routing
    path, the slot grid and the token-sum W2 included, with a shared expert."""
    _say(f"top_k={top_k} T={T} path={path}")
    _check_layer(synth.make_layer(6, num_experts=64, hidden=1024, intermediate=512, zipf=True,
                                  shared=True), T, top_k, path)


@pytest.mark.parametrize("T,path,top_k", [(1, "decode", 16), (3, "decode", 64), (40, "decode", 16),
                                          (9, "decode", 32), (20, "prefill", 64),
                                          (300, "prefill", 16), (100, "auto", 64)])
def test_many_experts_per_token(T, path, top_k):
    """top_k up to the entry points' limit of 64 (64 = every expert of the layer), with a shared
    expert: the selection rounds past 8, the block-routed decode kernels (the slot grid and the
    token-sum W2 take at most 8), the sum over more than 8 rows per token, and at prefill the
    certified top-k and the large-input align (4 800 and 6 500 slots)."""
    _say(f"top_k={top_k} T={T} path={path}")
    _check_layer(synth.make_layer(7, num_experts=64, hidden=1024, intermediate=512, zipf=True,
                                  shared=True), T, top_k, path)


@pytest.mark.parametrize("T,shared", [(4096, False), (4096, True), (8192, False)])
def test_prefill_batches_past_the_large_input_align(T, shared):
    """Prefill batches of 4 096 and 8 192 tokens (top-8, 64 experts, the hottest routed by
    nearly every token): 32 768, 36 864 and 65 536 slots through the layer call's many-workgroup
    align (its ranks and chunk counts in the workspace, the GEMMs' block order written beside
    the layout), past the 32 768 slots that the standalone align's two-kernel form holds."""
    _say(f"prefill T={T} shared={shared}")
    _check_layer(synth.make_layer(8, num_experts=64, hidden=512, intermediate=256, zipf=True,
                                  shared=shared), T, 8, "prefill")
