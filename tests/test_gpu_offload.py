"""GPU tests of the offloaded-expert path: slot cache with real copies, slot-pool expert sets,
and the per-layer predictor.

* A layer read from its HBM slots must give bit-identical output to the same layer read from a
  resident stack (same kernels, same bytes), for every path, after evictions and prefetches.
* Slot contents must equal the host blob of the expert the table names (byte-exact).
* The predictor's top-k must match the oracle's (predictor_ref); a position may differ only
  where the oracle's logits of the two experts involved are within 1e-4 relative of each other
  (a one-ulp difference of expf in SiLU can move one bf16 activation by one step).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mtp_amd import ops, synth
from mtp_amd.offload import OffloadedExperts, pack_blobs, routed_layer
from oracle import moe_ref
from tests.helpers import LAYER_RTOL, bf16_bits, experts_to_np, small_layer, to_gpu

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)


@pytest.fixture(scope="module")
def pooled():
    _say("offload: building 2-layer pool (E16 H512 I256, 10 slots)")
    layers = [to_gpu(small_layer(l, zipf=True)) for l in range(2)]
    pool = OffloadedExperts(2, 16, 512, 256, 10, group_size=128, device="cuda")
    for l, g in enumerate(layers):
        pool.store_layer(l, g.experts)
    torch.cuda.synchronize()
    yield layers, pool
    pool.close()


def _slot_bytes_ok(pool: OffloadedExperts, layer: int, experts, blobs: torch.Tensor) -> None:
    for e in set(int(v) for v in experts):
        s = pool.cache.slot_of(layer, e)
        assert s >= 0, f"expert {e} of layer {layer} not resident"
        assert torch.equal(pool.device_pool[layer, s], blobs[e]), (layer, e, s)


@pytest.mark.parametrize("path", ["decode", "prefill"])
def test_pooled_layer_matches_resident(pooled, path):
    layers, pool = pooled
    rng = np.random.default_rng(11)
    for step, T in enumerate((1, 2, 1, 2, 2, 1)):
        layer = step % 2
        g = layers[layer]
        _say(f"  pooled layer {layer} T={T} path={path}")
        x = synth.make_tokens(T, 512, seed=100 + step).cuda()
        ids, w, _, _ = ops.router_topk(x, g.router_w, 4, logit_bias=g.logit_bias)
        # unrelated prefetches first, so demand has to evict and refetch
        pool.prefetch(layer, rng.choice(16, size=3, replace=False).tolist())
        pool.demand(layer, ids.cpu().reshape(-1).tolist())
        got = ops.fused_experts(x, ids, w, pool.layer_experts(layer), path=path)
        want = ops.fused_experts(x, ids, w, g.experts, path=path)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        _slot_bytes_ok(pool, layer, ids.cpu().reshape(-1).tolist(), pack_blobs(g.experts))


def test_prefetch_then_demand_hits_and_bytes(pooled):
    layers, pool = pooled
    before = pool.stats()
    issued = pool.prefetch(1, [13, 14, 15])
    hits = pool.demand(1, [13, 14, 15])
    torch.cuda.synchronize()
    after = pool.stats()
    assert hits == 3
    assert after["prefetch_bytes"] - before["prefetch_bytes"] == issued * pool.blob
    _slot_bytes_ok(pool, 1, [13, 14, 15], pack_blobs(layers[1].experts))


def test_routed_layer_matches_oracle(pooled):
    layers, pool = pooled
    lay_cpu = small_layer(0, zipf=True)
    x = synth.make_tokens(2, 512, seed=77)
    out, ids_host = routed_layer(x.cuda(), layers[0].router_w, pool, 0, top_k=4,
                                 logit_bias=layers[0].logit_bias)
    torch.cuda.synchronize()
    ref, r_ids, _, _ = moe_ref.moe_layer_ref(bf16_bits(x), bf16_bits(lay_cpu.router_w),
                                             experts_to_np(lay_cpu.experts), top_k=4,
                                             logit_bias=lay_cpu.logit_bias.numpy())
    assert np.array_equal(ids_host.numpy(), r_ids)
    assert moe_ref.rel_err(out.float().cpu().numpy(), ref) <= LAYER_RTOL


@pytest.mark.parametrize("T,path", [(1, "decode"), (2, "decode"), (2, "prefill")])
def test_offload_layer_call_matches_resident_layer(pooled, T, path):
    """moe_offload_layer_v1 (router, ids to the host, demand, the experts from the slots,
    layer_done and the prefetch list in one call) gives the resident layer's ids and output
    bit for bit, counts the demand, and the prefetched experts that are resident afterwards
    hold their host bytes."""
    _say(f"offload layer call T={T} path={path}")
    layers, pool = pooled
    layer = 1
    g = layers[layer]
    x = synth.make_tokens(T, 512, seed=90 + T).cuda()
    before = pool.stats()
    out, ids_host = routed_layer(x, g.router_w, pool, layer, top_k=4, logit_bias=g.logit_bias,
                                 prefetch=[7, 8, 9], path=path)
    want, ids, _ = ops.moe_layer(x, g.router_w, g.experts, top_k=4, logit_bias=g.logit_bias,
                                 path=path, return_routing=True)
    torch.cuda.synchronize()
    after = pool.stats()
    assert np.array_equal(ids_host.numpy(), ids.cpu().numpy())
    assert torch.equal(out, want)
    assert after["demand_count"] - before["demand_count"] == T * 4
    _slot_bytes_ok(pool, layer, ids_host.reshape(-1).tolist(), pack_blobs(g.experts))
    issued = after["issued_fetch_count"] - before["issued_fetch_count"]
    skipped = after["prefetch_skipped_pinned_count"] - before["prefetch_skipped_pinned_count"]
    assert issued + skipped <= 3
    assert after["prefetch_bytes"] - before["prefetch_bytes"] == issued * pool.blob
    resident = [e for e in (7, 8, 9) if pool.cache.slot_of(layer, e) >= 0]
    _slot_bytes_ok(pool, layer, resident, pack_blobs(g.experts))


@pytest.mark.parametrize("where", ["pageable", "pinned_at_an_offset"])
def test_offload_layer_ids_reach_any_host_buffer(pooled, where):
    """The routed ids reach pageable host memory (a copy on the stream) and pinned memory at an
    offset into its allocation (written by the top-k kernel through the mapping) alike."""
    _say(f"offload layer ids into {where} memory")
    layers, pool = pooled
    layer, T = 0, 3
    g = layers[layer]
    x = synth.make_tokens(T, 512, seed=123).cuda()
    if where == "pageable":
        ids_buf = torch.full((T, 4), -7, dtype=torch.int32)
    else:
        big = torch.full((T * 4 + 40,), -7, dtype=torch.int32, pin_memory=True)
        ids_buf = big[13:13 + T * 4].view(T, 4)
    out, ids_host = routed_layer(x, g.router_w, pool, layer, top_k=4, logit_bias=g.logit_bias,
                                 ids_host=ids_buf, path="decode")
    want, ids, _ = ops.moe_layer(x, g.router_w, g.experts, top_k=4, logit_bias=g.logit_bias,
                                 path="decode", return_routing=True)
    torch.cuda.synchronize()
    assert ids_host.data_ptr() == ids_buf.data_ptr()
    assert np.array_equal(ids_host.numpy(), ids.cpu().numpy())
    assert torch.equal(out, want)
    if where != "pageable":
        assert bool((big[:13] == -7).all()) and bool((big[13 + T * 4:] == -7).all())


def test_offload_layer_refuses_device_or_mistyped_ids_buffers(pooled):
    """The cache's demand reads the routed ids on the host: an ids buffer in device memory or of
    another dtype is refused before any call."""
    layers, pool = pooled
    g = layers[0]
    x = synth.make_tokens(3, 512, seed=124).cuda()
    for buf in (torch.zeros(3, 4, dtype=torch.int32, device="cuda"),
                torch.zeros(3, 4, dtype=torch.int64)):
        with pytest.raises(ValueError, match="ids_host"):
            routed_layer(x, g.router_w, pool, 0, top_k=4, logit_bias=g.logit_bias,
                         ids_host=buf, path="decode")


@pytest.mark.parametrize("T,L,H,D,E,k", [(1, 3, 512, 256, 64, 16), (4, 2, 2048, 1024, 256, 16),
                                          (3, 1, 256, 64, 40, 5)])
def test_predictor_matches_oracle(T, L, H, D, E, k):
    _say(f"predictor T={T} L={L} H={H} D={D} E={E} k={k}")
    g = torch.Generator().manual_seed(T * 1000 + L)
    h = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(L, D, H, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(L, E, D, generator=g) * 0.02).to(torch.bfloat16)
    ids = ops.predictor_topk(h.cuda(), w1.cuda(), w2.cuda(), k).cpu().numpy()
    r_ids, r_logits = moe_ref.predictor_ref(bf16_bits(h), bf16_bits(w1), bf16_bits(w2), k)
    assert ids.shape == r_ids.shape
    for l in range(L):
        for t in range(T):
            for j in range(k):
                a, b = int(ids[l, t, j]), int(r_ids[l, t, j])
                if a != b:
                    la, lb = r_logits[l, t, a], r_logits[l, t, b]
                    assert abs(la - lb) <= 1e-4 * max(abs(lb), 1e-3), (l, t, j, a, b, la, lb)


def test_predictor_rejects_bad_shapes():
    h = torch.zeros(1, 64, dtype=torch.bfloat16, device="cuda")
    w1 = torch.zeros(2, 32, 64, dtype=torch.bfloat16, device="cuda")
    w2 = torch.zeros(3, 16, 32, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        ops.predictor_topk(h, w1, w2, 4)


@pytest.mark.parametrize("path", ["decode", "prefill"])
def test_nonresident_expert_is_dropped(pooled, path):
    """A pool view maps experts that are not resident to row -1: their slots contribute zero
    (never a read through a negative row)."""
    layers, pool = pooled
    layer = 1
    g = layers[layer]
    pool.demand(layer, [0, 1, 2, 3, 4, 5])
    absent = [e for e in range(16) if pool.cache.slot_of(layer, e) < 0]
    assert absent, "the 10-slot pool cannot hold all 16 experts"
    e_nr = absent[0]
    _say(f"  non-resident expert {e_nr} path={path}")
    T = 3
    ids = np.array([[0, 1, e_nr, 2], [e_nr, 3, 4, 5], [5, 4, 3, e_nr]], dtype=np.int32)
    w = np.full(ids.shape, 0.25, dtype=np.float32)
    x = synth.make_tokens(T, 512, seed=77)
    got = ops.fused_experts(x.cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(),
                            pool.layer_experts(layer), path=path)
    torch.cuda.synchronize()
    lay_cpu = small_layer(layer, zipf=True)
    ref = moe_ref.moe_layer_f32(bf16_bits(x), ids, w, experts_to_np(lay_cpu.experts),
                                dropped=frozenset({e_nr}))
    err = moe_ref.rel_err(got.float().cpu().numpy(), ref)
    _say(f"  rel_err={err:.3e}")
    assert np.isfinite(err) and err <= LAYER_RTOL


def test_prefetch_between_demand_and_kernels_keeps_demanded_slots(pooled):
    """demand -> prefetch -> kernels on one stream: the prefetch may not take a slot the demand
    published (the kernels that read it are enqueued after the prefetch's copies start), so the
    output equals the resident layer's and the demanded slots keep their experts."""
    layers, pool = pooled
    layer = 0
    g = layers[layer]
    x = synth.make_tokens(2, 512, seed=91).cuda()
    ids, w, _, _ = ops.router_topk(x, g.router_w, 4, logit_bias=g.logit_bias)
    demanded = sorted(set(ids.cpu().reshape(-1).tolist()))
    pool.demand(layer, demanded)
    slots = {e: pool.cache.slot_of(layer, e) for e in demanded}
    others = [e for e in range(16) if e not in demanded]
    pool.prefetch(layer, others)  # more experts than free slots: LRU pressure on every slot
    assert {e: pool.cache.slot_of(layer, e) for e in demanded} == slots
    got = ops.fused_experts(x, ids, w, pool.layer_experts(layer), path="decode")
    pool.layer_done(layer)
    want = ops.fused_experts(x, ids, w, g.experts, path="decode")
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    blobs = pack_blobs(g.experts)
    _slot_bytes_ok(pool, layer, demanded, blobs)
    # every prefetched expert that is resident holds its own bytes: the list was longer than the
    # unpinned slots, so some slots were filled twice within the one call
    _slot_bytes_ok(pool, layer, [e for e in others if pool.cache.slot_of(layer, e) >= 0], blobs)


def test_repeated_prefetches_into_one_slot_keep_the_last_experts_bytes():
    """Prefetch calls with no demand between them refill the same LRU slots: with one slot per
    layer every call overwrites it, and the slot must end with the bytes of the expert its table
    entry names (the copies into one slot run in issue order)."""
    E, H, I = 16, 512, 256
    g = to_gpu(small_layer(3))
    blobs = pack_blobs(g.experts)
    for slots in (1, 3):
        pool = OffloadedExperts(1, E, H, I, slots, group_size=128, device="cuda")
        try:
            pool.store_layer(0, g.experts)
            torch.cuda.synchronize()
            for rep in range(4):
                _say(f"  slots={slots} rep={rep}")
                pool.prefetch(0, [(5 * rep + i) % E for i in range(7)])
                pool.prefetch(0, [(3 * rep + 11 + i) % E for i in range(5)])
                torch.cuda.synchronize()
                resident = [e for e in range(E) if pool.cache.slot_of(0, e) >= 0]
                assert len(resident) == slots
                _slot_bytes_ok(pool, 0, resident, blobs)
        finally:
            pool.close()


def test_demand_of_a_prefetch_older_than_the_event_ring_is_on_time():
    """A prefetched expert first demanded after more prefetch calls than the handle keeps timing
    events for (1024): its own event has been re-recorded by a later call (here on another layer,
    still in flight when the demand is issued), so the check is skipped and the expert counts as
    on time, not as a ready-late miss measured against an unrelated copy."""
    E, H, I = 16, 512, 256
    g = to_gpu(small_layer(4))
    pool = OffloadedExperts(2, E, H, I, 2, group_size=128, device="cuda")
    try:
        pool.store_layer(0, g.experts)
        pool.store_layer(1, g.experts)
        torch.cuda.synchronize()
        pool.prefetch(0, [3])
        torch.cuda.synchronize()
        _say("  1100 prefetch calls on layer 1")
        for i in range(1100):  # each call issues one copy (two slots, three experts in turn)
            assert pool.prefetch(1, [i % 3]) == 1
        pool.demand(0, [3])
        pool.layer_done(0)
        torch.cuda.synchronize()
        st = pool.stats()
        assert st["demand_hit_count"] == 1 and st["used_fetch_count"] == 1
        assert st["ready_late_miss_count"] == 0, st
        _slot_bytes_ok(pool, 0, [3], pack_blobs(g.experts))
    finally:
        pool.close()


def test_store_loads_into_hbm_stacks_and_the_pinned_pool(tmp_path):
    """A written repacked store loaded two ways - load_layer (verified, HBM stacks) and
    OffloadedExperts.load_from_store (verified, straight into the pinned host pool) - gives the
    oracle's layer output; the pooled slots hold the same bytes as the resident stacks."""
    from mtp_amd.repack import RepackedMoeExpertStore
    from mtp_amd.repack.store import write_repacked_store
    E, H, I = 16, 512, 256
    lays = [small_layer(20 + l) for l in range(2)]
    tensors = {}
    for l, lay in enumerate(lays):
        t = {}
        for name, st in (("gate_proj", lay.experts.gate), ("up_proj", lay.experts.up),
                         ("down_proj", lay.experts.down)):
            t[f"experts.{name}.qweight"] = st.qweight
            t[f"experts.{name}.qzeros"] = st.qzeros
            t[f"experts.{name}.scales"] = st.scales
            t[f"experts.{name}.g_idx"] = (torch.arange(st.in_features, dtype=torch.int32) // 128).repeat(E, 1)
        tensors[l] = t
    write_repacked_store(tmp_path, tensors, num_experts=E)
    pool = OffloadedExperts(2, E, H, I, 6, group_size=128, device="cuda")
    try:
        with RepackedMoeExpertStore(tmp_path) as store:
            for l in range(2):
                _say(f"  store layer {l}")
                resident = store.load_layer(l, device="cuda")
                pool.load_from_store(store, l)
                x = synth.make_tokens(3, H, seed=90 + l)
                rng = np.random.default_rng(l)
                ids = np.stack([rng.choice(E, 2, replace=False) for _ in range(3)]).astype(np.int32)
                w = rng.uniform(0.2, 0.8, ids.shape).astype(np.float32)
                idt, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
                pool.demand(l, ids.reshape(-1).tolist())
                got_pool = ops.fused_experts(x.cuda(), idt, wt, pool.layer_experts(l), path="decode")
                pool.layer_done(l)
                got_res = ops.fused_experts(x.cuda(), idt, wt, resident, path="decode")
                torch.cuda.synchronize()
                assert torch.equal(got_pool, got_res)
                _slot_bytes_ok(pool, l, ids.reshape(-1).tolist(), pack_blobs(resident))
                ref = moe_ref.moe_layer_f32(bf16_bits(x), ids, w, experts_to_np(lays[l].experts))
                assert moe_ref.rel_err(got_res.float().cpu().numpy(), ref) <= LAYER_RTOL
    finally:
        pool.close()


def _hr_oracle_params(m):
    b = lambda t: bf16_bits(t)  # noqa: E731
    return {"enc_w": b(m.enc_w), "enc_b": m.enc_b.cpu().numpy(), "ln_w": b(m.ln_w),
            "ln_b": b(m.ln_b), "layer_emb": b(m.layer_emb), "delta_emb": b(m.delta_emb),
            "cls_w": b(m.cls_w), "cls_b": m.cls_b.cpu().numpy()}


def _ids_match_up_to_near_ties(got, want, logits, atol):
    g, w, lg = got.reshape(-1, got.shape[-1]), want.reshape(-1, want.shape[-1]), logits.reshape(-1, logits.shape[-1])
    for r in range(g.shape[0]):
        for j in range(g.shape[1]):
            a, b = int(g[r, j]), int(w[r, j])
            if a != b:
                assert abs(float(lg[r, a]) - float(lg[r, b])) <= atol, (r, j, a, b)


@pytest.mark.parametrize("scope", ["fixed", "layer"])
def test_hidden_residual_predictor_matches_oracle(scope):
    """The reference's HiddenResidualExpertPredictor at its default shape (hidden 2048, width
    256, 40 layers, 4 future deltas, 256 experts) on the HIP kernels against the oracle:
    residual and combined logits within bf16-activation tolerance, top-16 ids equal up to
    near-ties."""
    from mtp_amd.predictor import HiddenResidualExpertPredictor
    _say(f"hidden-residual predictor scope={scope}")
    m = HiddenResidualExpertPredictor(seed=5, learnable_residual_gamma=(scope == "layer"),
                                      residual_gamma_scope="layer" if scope == "layer" else "scalar",
                                      initial_residual_gamma=0.8)
    if scope == "layer":
        m.raw_residual_gamma.data.copy_(torch.linspace(-1.0, 1.0, 40, device="cuda"))
    g = torch.Generator().manual_seed(6)
    N = 5
    h = torch.randn(N, 2048, generator=g).to(torch.bfloat16)
    lid = torch.tensor([0, 39, 7, 7, 20], dtype=torch.int32)
    prior = torch.randn(N, 4, 256, generator=g)
    ids, out = m.predict_topk(h.cuda(), layer_ids=lid, k=16, prior=prior, fixed_scale=0.7,
                              return_logits=True)
    resid = m(h.cuda(), layer_ids=lid)
    torch.cuda.synchronize()
    p = _hr_oracle_params(m)
    per = None
    if scope == "layer":
        per = torch.nn.functional.softplus(torch.linspace(-1.0, 1.0, 40))[lid.long()].numpy()
    r_ids, r_out, r_res = moe_ref.hidden_residual_ref(bf16_bits(h), p, lid.numpy(), top_k=16,
                                                      prior=prior.numpy(), scale=0.7,
                                                      scale_per_example=per)
    atol = 5e-3
    assert np.max(np.abs(resid.cpu().numpy() - r_res)) <= atol
    assert np.max(np.abs(out.cpu().numpy() - r_out)) <= atol * 2
    _ids_match_up_to_near_ties(ids.cpu().numpy(), r_ids, r_out, 4 * atol)
    with pytest.raises(ValueError, match="layer_ids must have shape"):
        m(h.cuda(), layer_ids=lid[:2])


def test_hidden_residual_predictor_loads_a_reference_state_dict():
    """Parameters in the reference module's state_dict names: the forward then agrees with the
    same architecture built from torch's layers in fp32 (to bf16 accuracy)."""
    from mtp_amd.predictor import HiddenResidualExpertPredictor
    H, W, L, Fw, E = 512, 128, 6, 3, 64
    torch.manual_seed(3)
    enc = torch.nn.Sequential(torch.nn.Linear(H, W), torch.nn.SiLU(), torch.nn.LayerNorm(W))
    lemb, demb, cls = torch.nn.Embedding(L, W), torch.nn.Embedding(Fw, W), torch.nn.Linear(W, E)
    with torch.no_grad():  # bf16-representable parameters, as a bf16 checkpoint holds them
        for mod in (enc[0], enc[2], lemb, demb, cls):
            for prm in mod.parameters():
                prm.copy_(prm.to(torch.bfloat16).float())
    state = {"encoder.0.weight": enc[0].weight, "encoder.0.bias": enc[0].bias,
             "encoder.2.weight": enc[2].weight, "encoder.2.bias": enc[2].bias,
             "layer_embedding.weight": lemb.weight, "delta_embedding.weight": demb.weight,
             "classifier.weight": cls.weight, "classifier.bias": cls.bias}
    m = HiddenResidualExpertPredictor(hidden_size=H, num_experts=E, num_layers=L,
                                      future_window=Fw, width=W)
    m.load_reference_state_dict(state)
    h = torch.randn(4, H).to(torch.bfloat16)
    lid = torch.tensor([0, 5, 2, 2])
    got = m(h.cuda(), layer_ids=lid).cpu().numpy()
    with torch.no_grad():
        st = enc(h.float())
        ctx = st[:, None, :] + lemb(lid)[:, None, :] + demb(torch.arange(Fw))[None, :, :]
        want = cls(torch.nn.functional.silu(ctx)).numpy()
    assert moe_ref.rel_err(got, want) < 2e-2


def test_ready_late_first_demands_are_counted_from_event_times():
    """Prefetches still in flight when the layer demands them are ready-late (the copy completes
    after the demand's event); prefetches that completed first are not. The layer output stays
    exact either way (the demand waits for the copies)."""
    E, H, I = 16, 2048, 512
    ex = synth.make_experts(E, H, I, seed=77, device="cuda")
    pool = OffloadedExperts(1, E, H, I, 8, group_size=128, device="cuda")
    try:
        pool.store_layer(0, ex)
        torch.cuda.synchronize()
        # completed before the demand: not late
        pool.prefetch(0, [0, 1])
        torch.cuda.synchronize()
        pool.demand(0, [0, 1])
        pool.layer_done(0)
        torch.cuda.synchronize()
        st = pool.stats()
        assert st["ready_late_miss_count"] == 0 and st["demand_hit_count"] == 2
        # six 1.6 MB copies queued right before the demand: the later ones complete after it
        pool.prefetch(0, [2, 3, 4, 5, 6, 7])
        pool.demand(0, [2, 3, 4, 5, 6, 7])
        x = synth.make_tokens(1, H, seed=3).cuda()
        ids = torch.tensor([[2, 3, 4, 5, 6, 7]], dtype=torch.int32, device="cuda")
        w = torch.full((1, 6), 1.0 / 6, device="cuda")
        got = ops.fused_experts(x, ids, w, pool.layer_experts(0), path="decode")
        pool.layer_done(0)
        want = ops.fused_experts(x, ids, w, ex, path="decode")
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        st = pool.stats()
        _say(f"  ready-late {st['ready_late_miss_count']} of 6, wait {st['ready_late_wait_ns'] / 1e3:.1f} us")
        assert st["ready_late_miss_count"] >= 1 and st["ready_late_wait_ns"] > 0
        assert st["demand_hit_count"] == 8
    finally:
        pool.close()


def test_offload_decoder_at_the_full_config5_shape():
    """Config 5's loop at its own shape: two offloaded layers of H 2048 / I 512 / 256 experts
    with 64 HBM slots each, OffloadDecoder.step at batch 1 for several steps with predicted
    prefetch lists (the hidden-residual predictor) after every layer. Every step's per-layer
    output equals the resident layer's bit for bit, and the slot cache's counters equal one
    LRU oracle per layer (cache_manager.py:208-279) fed the same demanded ids and prefetch lists
    (the demand's slots, still pinned while the layer call prefetches, are the layer's most
    recently used, so with 64 slots the LRU victim is never one of them)."""
    from mtp_amd.offload import OffloadDecoder
    from mtp_amd.predictor import HiddenResidualExpertPredictor
    from oracle.cache_ref import LruCounters
    L, E, H, I, K, S = 2, 256, 2048, 512, 8, 64
    _say("config 5 full shape: building 2 layers")
    layers = [synth.make_layer(l, zipf=True, device="cuda") for l in range(L)]
    pool = OffloadedExperts(L, E, H, I, S, group_size=128, device="cuda")
    try:
        for l, g in enumerate(layers):
            pool.store_layer(l, g.experts)
        torch.cuda.synchronize()
        hr = HiddenResidualExpertPredictor(hidden_size=H, num_experts=E, num_layers=L, seed=9,
                                           device="cuda")
        dec = OffloadDecoder(pool, [g.router_w for g in layers], [g.logit_bias for g in layers],
                             top_k=K, predictor=hr, prefetch_k=16, path="decode")
        gen = torch.Generator(device="cuda")
        gen.manual_seed(17)
        xs = torch.randn(7, 1, H, generator=gen, device="cuda").to(torch.bfloat16)
        trace = []
        for t in range(6):
            _say(f"  step {t}")
            pre = dec.predict(xs[t + 1])
            outs = dec.step(xs[t], pre, trace=trace)
            for l, g in enumerate(layers):
                want = ops.moe_layer(xs[t], g.router_w, g.experts, top_k=K,
                                     logit_bias=g.logit_bias, path="decode")
                torch.cuda.synchronize()
                assert torch.equal(outs[l], want), (t, l)
        oracles = [LruCounters(S) for _ in range(L)]
        for layer, ids, pre, _ in trace:
            for e in ids:
                oracles[layer].demand(layer, e)
            for e in pre:
                oracles[layer].issue_prefetch(layer, e)
        st = pool.stats()
        want = {
            "issued_fetch_count": sum(o.issued for o in oracles),
            "used_fetch_count": sum(o.used for o in oracles),
            "unused_fetch_count": sum(o.unused() for o in oracles),
            "demand_count": sum(o.demand_count for o in oracles),
            "demand_hit_count": sum(o.hits for o in oracles),
            "demand_miss_count": sum(o.misses for o in oracles),
            "evicted_before_use_count": sum(o.evicted_before_use for o in oracles),
            "resident_count": sum(len(o.cache) for o in oracles),
        }
        for k, v in want.items():
            assert st[k] == v, (k, st[k], v)
        assert st["prefetch_skipped_pinned_count"] == 0
        assert st["demand_count"] == 6 * L * K and st["issued_fetch_count"] > 0
        _say(f"  hits {st['demand_hit_count']} of {st['demand_count']}, issued "
             f"{st['issued_fetch_count']}")
    finally:
        pool.close()


def test_offload_decoder_rechecks_replaced_routers_and_top_k():
    """OffloadDecoder caches each layer's call arguments between steps; a router or bias tensor
    replaced in `routers`/`biases`, or a new top_k, must be picked up by the next step (outputs
    equal the resident layers with the new arguments)."""
    from mtp_amd.offload import OffloadDecoder
    _say("offload decoder: replaced router, bias and top_k between steps")
    layers = [to_gpu(small_layer(l, zipf=True)) for l in range(2)]
    pool = OffloadedExperts(2, 16, 512, 256, 16, group_size=128, device="cuda")
    try:
        for l, g in enumerate(layers):
            pool.store_layer(l, g.experts)
        torch.cuda.synchronize()
        routers = [g.router_w for g in layers]
        biases = [g.logit_bias for g in layers]
        dec = OffloadDecoder(pool, routers, biases, top_k=4, path="decode")
        x = torch.randn(2, 512, device="cuda").to(torch.bfloat16)

        def check(top_k):
            outs = dec.step(x)
            for l, g in enumerate(layers):
                want = ops.moe_layer(x, dec.routers[l], g.experts, top_k=top_k,
                                     logit_bias=dec.biases[l], path="decode")
                torch.cuda.synchronize()
                assert torch.equal(outs[l], want), (l, top_k)

        check(4)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(5)
        dec.routers[1] = (torch.randn(16, 512, generator=gen, device="cuda") * 0.05).to(torch.bfloat16)
        dec.biases[0] = None
        check(4)
        dec.top_k = 2
        check(2)
    finally:
        pool.close()


def test_slot_cache_creation_error_leaves_no_state_behind():
    """A live cache on a device that does not exist is refused when its streams are set up; the
    partial set-up is released and the caller's current device is unchanged, so a valid cache
    created next works."""
    from mtp_amd import _lib
    from mtp_amd.offload import SlotCache
    dev_before = torch.cuda.current_device()
    host = torch.zeros(2 * 64, dtype=torch.uint8).pin_memory()
    pool = torch.zeros(2 * 64, dtype=torch.uint8, device="cuda")
    table = torch.full((2,), -1, dtype=torch.int32, device="cuda")
    with pytest.raises(_lib.MoeLibraryError, match="hipSetDevice"):
        SlotCache(1, 2, 2, 64, host_pool=host.data_ptr(), device_pool=pool.data_ptr(),
                  expert_row=table.data_ptr(), device=torch.cuda.device_count() + 3)
    assert torch.cuda.current_device() == dev_before
    cache = SlotCache(1, 2, 2, 64, host_pool=host.data_ptr(), device_pool=pool.data_ptr(),
                      expert_row=table.data_ptr(), device=dev_before)
    try:
        assert cache.demand(0, [1]) == 0
        torch.cuda.synchronize()
        assert cache.slot_of(0, 1) >= 0
    finally:
        cache.close()
    assert torch.cuda.current_device() == dev_before
