"""Repacked-store reader (mtp_amd/repack/store.py) against the reference's format
(tests/test_repack_qwen3_moe_gptq.py: stacking [E, ...], sha256 manifest, store slicing)."""

from __future__ import annotations

import pytest
import torch

from mtp_amd import synth
from mtp_amd.repack import RepackedMoeExpertStore, tensor_sha256
from mtp_amd.repack.store import write_repacked_store


def _layer_tensors(E=4, H=512, I=256):
    ex = synth.make_experts(E, H, I, seed=11)
    t = {}
    for name, st in (("gate_proj", ex.gate), ("up_proj", ex.up), ("down_proj", ex.down)):
        t[f"experts.{name}.qweight"] = st.qweight
        t[f"experts.{name}.qzeros"] = st.qzeros
        t[f"experts.{name}.scales"] = st.scales
        t[f"experts.{name}.g_idx"] = (torch.arange(st.in_features, dtype=torch.int32) // 128).repeat(E, 1)
    return t


def test_store_round_trip_slicing_and_hashes(tmp_path):
    tensors = _layer_tensors()
    write_repacked_store(tmp_path, {0: tensors, 3: tensors}, num_experts=4)
    with RepackedMoeExpertStore(tmp_path) as store:
        assert store.layers == (0, 3)
        assert store.num_experts == 4
        report = store.inspect(check_hashes=True)
        assert report["ok"], report
        q = store.get_expert_tensor(3, 2, "gate_proj", "qweight")
        assert torch.equal(q, tensors["experts.gate_proj.qweight"][2])
        info = store.tensor_info(0, "down_proj", "scales")
        assert info.shape == (4, 2, 512) and info.dtype == "float16"
        assert info.sha256 == tensor_sha256(tensors["experts.down_proj.scales"])
        with pytest.raises(IndexError):
            store.get_expert_tensor(0, 4, "gate_proj", "qweight")
        with pytest.raises(ValueError):
            store.tensor_key("o_proj", "qweight")
        with pytest.raises(KeyError):
            store.layer_path(1)


def test_store_detects_hash_mismatch(tmp_path):
    tensors = _layer_tensors()
    write_repacked_store(tmp_path, {0: tensors}, num_experts=4)
    bad = dict(tensors)
    bad["experts.up_proj.scales"] = tensors["experts.up_proj.scales"] * 2
    from safetensors.torch import save_file
    save_file(bad, str(tmp_path / "layer_00.safetensors"))
    report = RepackedMoeExpertStore(tmp_path).inspect(check_hashes=True)
    assert not report["ok"]
    assert [m["key"] for m in report["hash_mismatches"]] == ["experts.up_proj.scales"]


def test_synthetic_constants():
    assert synth.expert_bytes() == 1_634_304
    assert synth.prefill_flops(2048) == 103_079_215_104
    b = synth.zipf_logit_bias(256, seed=3000)
    assert b.shape == (256,) and torch.isfinite(b).all()


def test_load_layer_verifies_the_manifest_on_load(tmp_path):
    """load_layer / read_layer_tensors check every tensor against the manifest (shape, dtype,
    sha256) before anything is copied; a corrupted tensor is refused by name."""
    tensors = _layer_tensors()
    write_repacked_store(tmp_path, {0: tensors}, num_experts=4)
    with RepackedMoeExpertStore(tmp_path) as store:
        ex = store.load_layer(0, device="cpu")
        assert ex.group_size == 128 and ex.gate.num_rows == 4
        assert torch.equal(ex.down.qzeros, tensors["experts.down_proj.qzeros"])
    bad = dict(tensors)
    q = tensors["experts.gate_proj.qweight"].clone()
    q[1, 3, 5] ^= 1  # one bit of one packed word
    bad["experts.gate_proj.qweight"] = q
    from safetensors.torch import save_file
    save_file(bad, str(tmp_path / "layer_00.safetensors"))
    with RepackedMoeExpertStore(tmp_path) as store:
        with pytest.raises(ValueError, match="experts.gate_proj.qweight: sha256"):
            store.load_layer(0, device="cpu")
        assert store.load_layer(0, device="cpu", verify=False).gate.num_rows == 4
    bad["experts.gate_proj.qweight"] = q[:, :-1].contiguous()  # a shape the manifest does not list
    save_file(bad, str(tmp_path / "layer_00.safetensors"))
    with RepackedMoeExpertStore(tmp_path) as store:
        with pytest.raises(ValueError, match="shape"):
            store.read_layer_tensors(0, verify=False)
