"""The reference's repack API (load_topk_expert_mlp / TopKExpertMlp / SingleExpertMlp /
dequantize_repacked_projection) on the HIP kernels, read from an on-disk repacked store.
Mirrors tests/test_gptq_unpack.py:85-153 and scripts/smoke_topk_expert_mlp.py:65-119."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mtp_amd import synth
from mtp_amd.repack import (
    RepackedMoeExpertStore,
    dequantize_repacked_projection,
    load_single_expert_mlp,
    load_topk_expert_mlp,
)
from mtp_amd.repack.store import write_repacked_store
from oracle import gptq_ref, moe_ref
from tests.helpers import LAYER_RTOL, bf16_bits, experts_to_np, f16_bits

pytestmark = pytest.mark.gpu

E, H, I = 8, 512, 256


@pytest.fixture(scope="module")
def store_dir(tmp_path_factory):
    ex = synth.make_experts(E, H, I, seed=21)
    t = {}
    for name, st in (("gate_proj", ex.gate), ("up_proj", ex.up), ("down_proj", ex.down)):
        t[f"experts.{name}.qweight"] = st.qweight
        t[f"experts.{name}.qzeros"] = st.qzeros
        t[f"experts.{name}.scales"] = st.scales
        t[f"experts.{name}.g_idx"] = (torch.arange(st.in_features, dtype=torch.int32) // 128).repeat(E, 1)
    d = tmp_path_factory.mktemp("repacked")
    write_repacked_store(d, {0: t}, num_experts=E)
    return d, ex


def test_dequantize_repacked_projection_bit_exact(store_dir):
    d, ex = store_dir
    with RepackedMoeExpertStore(d) as store:
        got = dequantize_repacked_projection(store, layer=0, expert=5, projection="down_proj",
                                             device="cuda")
    want = gptq_ref.dequant_bf16_bits(ex.down.qweight[5].numpy(), ex.down.qzeros[5].numpy(),
                                      f16_bits(ex.down.scales[5]))
    assert np.array_equal(bf16_bits(got), want)


def test_topk_expert_mlp_weighted_sum(store_dir):
    d, ex = store_dir
    with RepackedMoeExpertStore(d) as store:
        mlp = load_topk_expert_mlp(store, layer=0, expert_ids=[3, 1, 3], device="cuda")
    assert mlp.loaded_expert_ids == (1, 3)
    assert mlp.hidden_size == H and mlp.intermediate_size == I
    x = synth.make_tokens(2 * 3, H, seed=8)
    ids = torch.tensor([3, 1], dtype=torch.long)
    w = torch.tensor([0.25, 0.75], dtype=torch.bfloat16)
    out = mlp(x.view(2, 3, H).cuda(), ids, w.cuda())
    assert out.shape == (2, 3, H) and out.dtype == torch.bfloat16
    ids_np = np.array([[3, 1]] * 6, dtype=np.int32)
    w_np = np.array([[0.25, 0.75]] * 6, dtype=np.float32)
    ref = moe_ref.moe_layer_f32(bf16_bits(x), ids_np, w_np, experts_to_np(ex))
    assert moe_ref.rel_err(out.view(6, H).float().cpu().numpy(), ref) <= LAYER_RTOL
    with pytest.raises(KeyError):
        mlp(x.cuda(), torch.tensor([2]), torch.tensor([1.0]))
    with pytest.raises(ValueError):
        mlp(x.cuda(), ids.view(1, 2), w.view(1, 2))


def test_single_expert_mlp(store_dir):
    d, ex = store_dir
    with RepackedMoeExpertStore(d) as store:
        mlp = load_single_expert_mlp(store, layer=0, expert=6, device="cuda")
    x = synth.make_tokens(5, H, seed=9)
    out = mlp(x.cuda())
    ref = moe_ref.moe_layer_f32(bf16_bits(x), np.full((5, 1), 6, np.int32), np.ones((5, 1), np.float32),
                                experts_to_np(ex))
    assert moe_ref.rel_err(out.float().cpu().numpy(), ref) <= LAYER_RTOL
    with pytest.raises(ValueError):
        mlp(torch.zeros(2, H + 8, dtype=torch.bfloat16, device="cuda"))
