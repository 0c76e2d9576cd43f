"""Router-trace payload helpers (mtp_amd.tracing): module resolution, token selection, routing
weights, loading and manifests. Expected values follow from how each synthetic payload is
built; the GPU replay of the trace smoke harness is in test_gpu_api.py."""

from __future__ import annotations

import json

import pytest
import torch

from mtp_amd.tracing import (load_trace_payload, resolve_router_module_name,
                             resolve_trace_sample, scores_to_router_weights, select_router_topk,
                             select_trace_hidden_token)

MODULES = ["model.layers.0.mlp.gate", "model.layers.1.mlp.gate", "model.layers.10.mlp.gate",
           "model.layers.1.mlp.shared_expert_gate"]


def _payload(B=2, T=3, k=4, calls=2, with_scores=True):
    g = torch.Generator().manual_seed(5)
    topk = {m: [torch.randint(0, 64, (B, T, k), generator=g) for _ in range(calls)]
            for m in MODULES}
    p = {"router_topk": topk, "last_hidden_state": torch.randn(B, T, 16, generator=g)}
    if with_scores:
        p["router_scores"] = {m: [torch.randn(B, T, k, generator=g) for _ in range(calls)]
                              for m in MODULES}
    return p


def test_router_module_of_a_layer():
    names = {m: None for m in MODULES}
    assert resolve_router_module_name(names, layer=1) == "model.layers.1.mlp.gate"
    assert resolve_router_module_name(names, layer=10) == "model.layers.10.mlp.gate"
    assert resolve_router_module_name(names) == sorted(MODULES)[0]
    assert resolve_router_module_name(names, module_name=MODULES[3]) == MODULES[3]
    with pytest.raises(KeyError):
        resolve_router_module_name(names, layer=7)
    with pytest.raises(KeyError):
        resolve_router_module_name(names, module_name="model.layers.2.mlp.gate")
    # the looser match: one "mlp.gate" module under "layers.3."
    assert resolve_router_module_name({"x.layers.3.mlp.gate.proj": 0}, layer=3) == \
        "x.layers.3.mlp.gate.proj"


def test_select_token_ids_and_softmax_weights():
    p = _payload()
    sel = select_router_topk(p, layer=1, call_index=1, batch_index=1, token_index=-1)
    want_ids = p["router_topk"]["model.layers.1.mlp.gate"][1][1, 2]
    want_scores = p["router_scores"]["model.layers.1.mlp.gate"][1][1, 2]
    assert sel.module_name == "model.layers.1.mlp.gate"
    assert torch.equal(sel.expert_ids, want_ids) and sel.expert_ids.dtype == torch.long
    assert torch.equal(sel.raw_scores, want_scores)
    assert torch.allclose(sel.expert_weights, torch.softmax(want_scores, -1))
    assert abs(float(sel.expert_weights.sum()) - 1.0) < 1e-6
    assert (sel.call_index, sel.batch_index, sel.token_index) == (1, 1, -1)
    two = select_router_topk(p, layer=1, call_index=1, batch_index=1, token_index=2, top_k=2)
    assert torch.equal(two.expert_ids, want_ids[:2])
    assert torch.allclose(two.expert_weights, torch.softmax(want_scores[:2], -1))


@pytest.mark.parametrize("mode", ["raw", "identity", "uniform", "equal", "SoftMax"])
def test_score_modes(mode):
    s = torch.tensor([2.0, -1.0, 0.5])
    w = scores_to_router_weights(s, mode=mode)
    if mode in ("raw", "identity"):
        assert torch.equal(w, s)
    elif mode in ("uniform", "equal"):
        assert torch.equal(w, torch.full((3,), 1.0 / 3))
    else:
        assert torch.allclose(w, torch.softmax(s, -1))
    assert w.dtype == torch.float32
    with pytest.raises(ValueError):
        scores_to_router_weights(s, mode="top1")
    with pytest.raises(ValueError):
        scores_to_router_weights(s.view(1, 3))


def test_equal_weights_without_scores_and_lower_rank_calls():
    p = _payload(with_scores=False)
    sel = select_router_topk(p, module_name=MODULES[0], token_index=1)
    assert sel.raw_scores is None
    assert torch.equal(sel.expert_weights, torch.full((4,), 0.25))
    q = {"router_topk": {"m.layers.0.mlp.gate": [torch.tensor([[3, 1], [5, 2]]),
                                                 torch.tensor([7, 8, 9])]}}
    assert select_router_topk(q, token_index=1).expert_ids.tolist() == [5, 2]       # [T, k]
    assert select_router_topk(q, call_index=-1).expert_ids.tolist() == [7, 8, 9]    # [k]


def test_selection_errors():
    p = _payload()
    with pytest.raises(KeyError):
        select_router_topk({"router_topk": {}})
    with pytest.raises(IndexError):
        select_router_topk(p, layer=0, call_index=2)
    with pytest.raises(IndexError):
        select_router_topk(p, layer=0, batch_index=-3)
    with pytest.raises(ValueError):
        select_router_topk({"router_topk": {"m": []}})
    with pytest.raises(ValueError):
        select_router_topk({"router_topk": {"m": [torch.zeros(1, 1, 1, 2, dtype=torch.long)]}})


def test_hidden_token_keeps_the_payload_rank():
    p = _payload()
    h = select_trace_hidden_token(p, batch_index=1, token_index=-1)
    assert h.shape == (1, 1, 16) and torch.equal(h[0, 0], p["last_hidden_state"][1, 2])
    h2 = select_trace_hidden_token({"last_hidden_state": p["last_hidden_state"][0]}, token_index=2)
    assert h2.shape == (1, 16) and torch.equal(h2[0], p["last_hidden_state"][0, 2])
    with pytest.raises(KeyError):
        select_trace_hidden_token({})
    with pytest.raises(ValueError):
        select_trace_hidden_token({"last_hidden_state": torch.zeros(16)})


class _NotATensor:
    pass


def test_payload_files_and_manifests(tmp_path):
    p = _payload()
    f = tmp_path / "samples" / "s0.pt"
    f.parent.mkdir()
    torch.save(p, f)
    got = load_trace_payload(f)
    assert torch.equal(got["last_hidden_state"], p["last_hidden_state"])
    assert sorted(got["router_topk"]) == sorted(MODULES)
    torch.save([1, 2], tmp_path / "list.pt")
    with pytest.raises(TypeError):
        load_trace_payload(tmp_path / "list.pt")
    torch.save({"obj": _NotATensor()}, tmp_path / "obj.pt")
    with pytest.raises(Exception):  # the safe loader refuses pickled objects
        load_trace_payload(tmp_path / "obj.pt")
    man = tmp_path / "manifest.jsonl"
    man.write_text("\n" + json.dumps({"path": "samples/s0.pt"}) + "\n")
    assert resolve_trace_sample(manifest_path=man) == f.resolve()
    assert resolve_trace_sample(sample_path=f, manifest_path=man) == f.resolve()
    with pytest.raises(ValueError):
        resolve_trace_sample()
    with pytest.raises(FileNotFoundError):
        resolve_trace_sample(sample_path=tmp_path / "missing.pt")
    (tmp_path / "empty.jsonl").write_text("\n")
    with pytest.raises(RuntimeError):
        resolve_trace_sample(manifest_path=tmp_path / "empty.jsonl")
    (tmp_path / "bad.jsonl").write_text(json.dumps({"path": "nope.pt"}) + "\n")
    with pytest.raises(FileNotFoundError):
        resolve_trace_sample(manifest_path=tmp_path / "bad.jsonl")
