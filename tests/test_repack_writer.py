"""The repacker (Qwen3-MoE GPTQ snapshot -> expert store) and the store reading its output.

Scenarios of the reference's tests/test_repack_qwen3_moe_gptq.py:15-126 (stacking, random
slice verification, store inspection and slicing on a one-shard, two-expert snapshot), then
GPTQ-shaped layers over two shards, the summary, and the error paths of
src/mtp_expert_prefetch/repack/qwen3_moe_gptq.py:120-140, 201-225.
"""

from __future__ import annotations

import json

import pytest
import torch
from safetensors.torch import load_file, save_file

from mtp_amd.repack.qwen3_moe_gptq import (
    load_repack_manifest,
    parse_layers,
    repack_qwen3_moe_gptq,
    verify_random_repacked_slices,
)
from mtp_amd.repack.store import KINDS, PROJECTIONS, RepackedMoeExpertStore, tensor_sha256


def _key(layer: int, expert: int, proj: str, kind: str) -> str:
    return f"model.language_model.layers.{layer}.mlp.experts.{expert}.{proj}.{kind}"


def _snapshot(root, tensors: dict[str, torch.Tensor], shards: int = 1) -> None:
    """Write tensors as a sharded snapshot with its index (key i goes to shard i % shards)."""
    root.mkdir(parents=True, exist_ok=True)
    names = [f"model-{i + 1:05d}-of-{shards:05d}.safetensors" for i in range(shards)]
    parts: list[dict[str, torch.Tensor]] = [{} for _ in range(shards)]
    weight_map = {}
    for i, (k, v) in enumerate(sorted(tensors.items())):
        parts[i % shards][k] = v
        weight_map[k] = names[i % shards]
    for name, part in zip(names, parts):
        save_file(part, str(root / name))
    (root / "model.safetensors.index.json").write_text(
        json.dumps({"metadata": {"total_size": 1}, "weight_map": weight_map}), encoding="utf-8")


def _toy(fill) -> dict[str, torch.Tensor]:
    return {_key(0, e, p, k): fill(e, k) for e in range(2) for p in PROJECTIONS for k in KINDS}


def test_repack_stacks_experts(tmp_path):
    src = _toy(lambda e, k: torch.full((2, 3), e + len(k), dtype=torch.float32))
    _snapshot(tmp_path / "snap", src)
    manifest = repack_qwen3_moe_gptq(tmp_path / "snap", tmp_path / "out", layers="0",
                                     num_experts=2, verify=True)
    records = [json.loads(line) for line in manifest.read_text(encoding="utf-8").splitlines()]
    assert len(records) == 1
    assert records[0]["num_source_tensors"] == 24
    assert records[0]["num_output_tensors"] == 12
    out = load_file(str(tmp_path / "out" / "layer_00.safetensors"))
    assert out["experts.gate_proj.qweight"].shape == (2, 2, 3)
    assert torch.equal(out["experts.gate_proj.qweight"][1], src[_key(0, 1, "gate_proj", "qweight")])


def test_verify_random_repacked_slices(tmp_path):
    src = _toy(lambda e, k: torch.arange(6, dtype=torch.float32).reshape(2, 3) + e)
    _snapshot(tmp_path / "snap", src)
    repack_qwen3_moe_gptq(tmp_path / "snap", tmp_path / "out", layers="0", num_experts=2)
    res = verify_random_repacked_slices(tmp_path / "snap", tmp_path / "out", samples=16, seed=7,
                                        num_experts=2)
    assert res["ok"] is True
    assert res["samples_checked"] == 16


def test_store_inspects_and_slices_the_repacked_output(tmp_path):
    src = _toy(lambda e, k: torch.arange(6, dtype=torch.int32).reshape(2, 3) + e)
    _snapshot(tmp_path / "snap", src)
    repack_qwen3_moe_gptq(tmp_path / "snap", tmp_path / "out", layers="0", num_experts=2)
    with RepackedMoeExpertStore(tmp_path / "out") as store:
        res = store.inspect()
        assert res["ok"] is True
        assert res["num_layers"] == 1
        assert res["total_output_tensors"] == 12
        info = store.tensor_info(0, "gate_proj", "qweight")
        assert info.shape == (2, 2, 3)
        assert info.dtype == "int32"
        assert torch.equal(store.get_expert_tensor(0, 1, "gate_proj", "qweight"),
                           src[_key(0, 1, "gate_proj", "qweight")])


def _gptq_layer(layer: int, E: int, H: int, I: int, G: int) -> dict[str, torch.Tensor]:
    """Per-expert GPTQ tensors of one layer in the checkpoint's shapes and dtypes."""
    g = torch.Generator().manual_seed(100 + layer)
    out = {}
    for e in range(E):
        for proj, (K, N) in (("gate_proj", (H, I)), ("up_proj", (H, I)), ("down_proj", (I, H))):
            out[_key(layer, e, proj, "qweight")] = torch.randint(
                -2**31, 2**31 - 1, (K // 8, N), generator=g, dtype=torch.int32)
            out[_key(layer, e, proj, "qzeros")] = torch.randint(
                -2**31, 2**31 - 1, (K // G, N // 8), generator=g, dtype=torch.int32)
            out[_key(layer, e, proj, "scales")] = (torch.rand(K // G, N, generator=g) * 0.01).to(
                torch.float16)
            out[_key(layer, e, proj, "g_idx")] = torch.arange(K, dtype=torch.int32) // G
    return out


def test_gptq_layers_over_two_shards_read_back_through_the_store(tmp_path):
    E, H, I, G = 4, 256, 128, 64
    src = {**_gptq_layer(0, E, H, I, G), **_gptq_layer(1, E, H, I, G), **_gptq_layer(3, E, H, I, G)}
    src["model.language_model.layers.0.mlp.gate.weight"] = torch.zeros(E, H)  # not an expert key
    _snapshot(tmp_path / "snap", src, shards=2)
    repack_qwen3_moe_gptq(tmp_path / "snap", tmp_path / "out", layers="0-1", num_experts=E,
                          verify=True)
    summary = json.loads((tmp_path / "out" / "summary.json").read_text(encoding="utf-8"))
    assert summary["layers"] == [0, 1] and summary["num_layers"] == 2
    assert summary["total_source_tensors"] == 2 * 12 * E
    assert summary["total_output_tensors"] == 24
    assert summary["reduction_factor"] == pytest.approx(E)
    assert summary["projections"] == list(PROJECTIONS) and summary["kinds"] == list(KINDS)
    records = load_repack_manifest(tmp_path / "out")
    rec = records[1]["tensors"]["experts.down_proj.scales"]
    assert rec["shape"] == [E, I // G, H] and rec["dtype"] == "float16"
    assert rec["source_count"] == E and rec["source_shape"] == [I // G, H]
    assert rec["source_key_template"] == "model.language_model.layers.1.mlp.experts.{expert}.down_proj.scales"
    with RepackedMoeExpertStore(tmp_path / "out") as store:
        assert store.inspect(check_hashes=True)["ok"] is True
        for layer in (0, 1):
            for e in range(E):
                for proj in PROJECTIONS:
                    for kind in KINDS:
                        got = store.get_expert_tensor(layer, e, proj, kind)
                        assert torch.equal(got, src[_key(layer, e, proj, kind)])
        stacked = store.get_fused_tensor(1, "gate_proj", "qweight")
        assert tensor_sha256(stacked) == records[1]["tensors"]["experts.gate_proj.qweight"]["sha256"]
    res = verify_random_repacked_slices(tmp_path / "snap", tmp_path / "out", samples=64, seed=3)
    assert res["ok"] and res["num_experts"] == E and res["layers"] == [0, 1]


def test_verify_reports_a_tampered_slice(tmp_path):
    src = _toy(lambda e, k: torch.arange(6, dtype=torch.int32).reshape(2, 3) + 10 * e)
    _snapshot(tmp_path / "snap", src)
    repack_qwen3_moe_gptq(tmp_path / "snap", tmp_path / "out", layers="0", num_experts=2)
    path = tmp_path / "out" / "layer_00.safetensors"
    t = load_file(str(path))
    for k in t:
        t[k] = t[k].clone()
        t[k][1] += 1
    save_file(t, str(path))
    res = verify_random_repacked_slices(tmp_path / "snap", tmp_path / "out", samples=32, seed=1,
                                        fail_fast=False)
    assert not res["ok"]
    assert res["samples_checked"] == 32
    assert all(f["expert"] == 1 and f["source_sha256"] != f["repacked_slice_sha256"]
               for f in res["failures"])


def test_repack_errors(tmp_path):
    src = _toy(lambda e, k: torch.zeros(2, 3))
    del src[_key(0, 1, "up_proj", "scales")]
    _snapshot(tmp_path / "snap", src)
    with pytest.raises(RuntimeError, match="missing 1 experts"):
        repack_qwen3_moe_gptq(tmp_path / "snap", tmp_path / "out", num_experts=2)
    (tmp_path / "out2").mkdir()
    (tmp_path / "out2" / "manifest.jsonl").write_text("{}\n", encoding="utf-8")
    with pytest.raises(FileExistsError):
        repack_qwen3_moe_gptq(tmp_path / "snap", tmp_path / "out2", num_experts=1)
    with pytest.raises(FileNotFoundError):
        repack_qwen3_moe_gptq(tmp_path / "nowhere", tmp_path / "out3")
    with pytest.raises(ValueError, match="descending"):
        parse_layers("3-1", [1, 2, 3])
    with pytest.raises(ValueError, match="not present"):
        parse_layers("0,7", [0, 1])
    assert parse_layers(" 2, 0-1 ,", [0, 1, 2, 3]) == [0, 1, 2]
    assert parse_layers(None, [4, 5]) == [4, 5]
