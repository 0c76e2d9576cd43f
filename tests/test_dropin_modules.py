"""Host-side structure of the drop-in expert modules (no GPU needed).

The reference's harnesses find the device with next(mlp.parameters(), next(mlp.buffers()))
(scripts/smoke_topk_expert_mlp.py:92) and move modules with .to(); the reference modules keep
their weights as non-persistent buffers (gptq_unpack.py:237-239). The int4 modules here hold
their GPTQ stacks the same way.
"""

from __future__ import annotations

import pytest
import torch

from mtp_amd import synth
from mtp_amd.repack import (
    GptqProjectionTensors,
    QuantizedExpertWeights,
    SingleExpertMlp,
    SingleExpertWeights,
    TopKExpertMlp,
)

H, I, E = 256, 128, 4


def _quantized(e: int) -> QuantizedExpertWeights:
    ex = synth.make_experts(E, H, I, seed=5)
    projs = {}
    for name, st in (("gate_proj", ex.gate), ("up_proj", ex.up), ("down_proj", ex.down)):
        g = torch.arange(st.in_features, dtype=torch.int32) // 128
        projs[name] = GptqProjectionTensors(st.qweight[e], st.qzeros[e], st.scales[e], g)
    return QuantizedExpertWeights(projs["gate_proj"], projs["up_proj"], projs["down_proj"], 128)


def test_topk_module_exposes_buffers_for_the_device_probe():
    mlp = TopKExpertMlp({3: _quantized(3), 1: _quantized(1)})
    dev = next(mlp.parameters(), next(mlp.buffers())).device
    assert dev.type == "cpu"
    names = {n for n, _ in mlp.named_buffers()}
    assert {"gate_proj_qweight", "up_proj_qzeros", "down_proj_scales"} <= names
    assert mlp.gate_proj_qweight.shape == (2, H // 8, I)
    assert mlp.loaded_expert_ids == (1, 3)
    assert (mlp.hidden_size, mlp.intermediate_size) == (H, I)
    # non-persistent, like the reference's dense buffers
    assert mlp.state_dict() == {}
    # rows are stacked in ascending id order
    assert torch.equal(mlp.down_proj_qweight[1], _quantized(3).down_proj.qweight)
    assert set(mlp.experts) == {"1", "3"}


def test_module_moves_rebuild_the_kernel_view():
    mlp = TopKExpertMlp({0: _quantized(0)})
    view = mlp.int4_experts()
    assert view is mlp.int4_experts()
    mlp.to(torch.device("cpu"))
    assert mlp._view is None
    assert mlp.int4_experts().gate.qweight.data_ptr() == mlp.gate_proj_qweight.data_ptr()


def test_forward_without_a_rocm_device_fails_loudly(monkeypatch):
    """Host modules and inputs are staged to a ROCm device; with none available the forward
    raises (there is no CPU path), and shape errors come first, as in the reference."""
    mlp = SingleExpertMlp(_quantized(2))
    with pytest.raises(ValueError, match="last dim"):
        mlp(torch.zeros(1, H + 8, dtype=torch.bfloat16))
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        mlp(torch.zeros(1, H, dtype=torch.bfloat16))


def test_dense_single_expert_weights_are_refused_with_a_message():
    dense = SingleExpertWeights(torch.zeros(I, H), torch.zeros(I, H), torch.zeros(H, I))
    with pytest.raises(TypeError, match="QuantizedExpertWeights"):
        SingleExpertMlp(dense)
    with pytest.raises(TypeError, match="QuantizedExpertWeights"):
        TopKExpertMlp({0: dense})


def test_dtypes_follow_the_reference_names():
    assert SingleExpertMlp(_quantized(0), dtype="fp16").compute_dtype == torch.float16
    assert SingleExpertMlp(_quantized(0), dtype="float32").compute_dtype == torch.float32
    single = SingleExpertMlp(_quantized(0), dtype="fp32")
    assert TopKExpertMlp({0: single}).compute_dtype == torch.float32
    with pytest.raises(ValueError, match="Unsupported dtype"):
        SingleExpertMlp(_quantized(0), dtype="int8")


def test_topk_module_validation_messages():
    with pytest.raises(ValueError, match="at least one expert"):
        TopKExpertMlp({})
    small = _quantized(0)
    other = synth.make_experts(1, H, 2 * I, seed=6)
    g = torch.arange(H, dtype=torch.int32) // 128
    g2 = torch.arange(2 * I, dtype=torch.int32) // 128
    big = QuantizedExpertWeights(
        GptqProjectionTensors(other.gate.qweight[0], other.gate.qzeros[0], other.gate.scales[0], g),
        GptqProjectionTensors(other.up.qweight[0], other.up.qzeros[0], other.up.scales[0], g),
        GptqProjectionTensors(other.down.qweight[0], other.down.qzeros[0], other.down.scales[0], g2))
    with pytest.raises(ValueError, match="share dimensions"):
        TopKExpertMlp({0: small, 1: big})
