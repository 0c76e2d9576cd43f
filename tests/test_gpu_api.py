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


def test_topk_expert_mlp_with_no_ids_and_with_more_than_64(store_dir):
    """The reference sums the listed experts one after another from zeros
    (gptq_unpack.py:318-326): no ids give zeros, and any number of ids is summed (the
    kernels take 64 experts per token per call; longer lists are summed in chunks)."""
    d, ex = store_dir
    with RepackedMoeExpertStore(d) as store:
        mlp = load_topk_expert_mlp(store, layer=0, expert_ids=list(range(E)), device="cuda")
    x = synth.make_tokens(5, H, seed=9)
    none = mlp(x.cuda(), torch.empty(0, dtype=torch.long), torch.empty(0))
    assert none.shape == (5, H) and not bool(none.any())
    rng = np.random.default_rng(4)
    ids_np = rng.integers(0, E, 150).astype(np.int32)
    w_np = rng.uniform(0.001, 0.01, 150).astype(np.float32)
    out = mlp(x.cuda(), torch.from_numpy(ids_np).long(), torch.from_numpy(w_np).cuda())
    # the module casts the weights to the input's dtype (bf16) first, as the reference does
    w_bf = torch.from_numpy(w_np).to(torch.bfloat16).float().numpy()
    ref = moe_ref.moe_layer_f32(bf16_bits(x), np.tile(ids_np, (5, 1)), np.tile(w_bf, (5, 1)),
                                experts_to_np(ex))
    assert moe_ref.rel_err(out.float().cpu().numpy(), ref) <= LAYER_RTOL


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


@pytest.mark.parametrize("dtype_name", ["bf16", "fp16", "fp32"])
def test_topk_harness_call_sequence(store_dir, dtype_name):
    """The call sequence of the reference's top-k smoke harness
    (scripts/smoke_topk_expert_mlp.py:65-119): resolve the dtype name, open the store as a
    context manager, load the deduplicated experts, find the device through
    next(parameters(), next(buffers())), draw [batch, seq, hidden] inputs in that dtype, call
    the module under inference_mode with CPU long ids and device weights of the same dtype,
    then read the reported fields. The output is checked against the oracle."""
    from mtp_amd.repack import resolve_torch_dtype
    d, ex = store_dir
    target = resolve_torch_dtype(dtype_name)
    expert_ids = [4, 0, 7, 4]
    expert_weights = [0.4, 0.3, 0.2, 0.1]
    torch.manual_seed(0)
    with RepackedMoeExpertStore(d) as store:
        mlp = load_topk_expert_mlp(store, layer=0, expert_ids=expert_ids, bits=4, dtype=target,
                                   device="cuda")
    device = next(mlp.parameters(), next(mlp.buffers())).device
    assert device.type == "cuda"
    x = torch.randn(2, 3, mlp.hidden_size, device=device, dtype=target)
    ids = torch.tensor(expert_ids, dtype=torch.long)
    weights = torch.tensor(expert_weights, dtype=target, device=device)
    with torch.inference_mode():
        out = mlp(x, ids, weights)
    assert bool(torch.isfinite(out).all().item())
    assert list(mlp.loaded_expert_ids) == [0, 4, 7]
    assert out.shape == x.shape and out.dtype == target
    assert (mlp.hidden_size, mlp.intermediate_size) == (H, I)
    # oracle: the kernels take bf16 activations, so the oracle input is the input rounded to
    # bf16; the routing weights are the harness's weights in its dtype
    xb = x.reshape(6, H).to(torch.bfloat16)
    w_np = np.tile(weights.float().cpu().numpy(), (6, 1))
    ref = moe_ref.moe_layer_f32(bf16_bits(xb), np.tile(np.array(expert_ids, np.int32), (6, 1)),
                                w_np, experts_to_np(ex))
    err = moe_ref.rel_err(out.reshape(6, H).float().cpu().numpy(), ref)
    print(f"  {dtype_name}: rel_err={err:.3e}", flush=True)
    assert err <= LAYER_RTOL
    # the same module moved to the CPU runs from its host buffers (staged to the GPU, result on
    # the host, same bits), and moved back runs again from its buffers
    mlp.to("cpu")
    assert next(mlp.buffers()).device.type == "cpu"
    with torch.inference_mode():
        on_host = mlp(x.cpu(), ids, weights.cpu())
    assert on_host.device.type == "cpu" and torch.equal(on_host, out.cpu())
    mlp.to(device)
    with torch.inference_mode():
        again = mlp(x, ids, weights)
    assert torch.equal(again, out)


@pytest.mark.parametrize("dtype_name", ["bf16", "fp16", "fp32"])
def test_single_expert_harness_call_sequence(store_dir, dtype_name):
    """The call sequence of the reference's single-expert smoke harness
    (scripts/smoke_single_expert_mlp.py:43-87): load one expert, draw inputs on
    mlp.gate_proj.device in mlp.gate_proj.dtype, run it, and report the projection shapes.
    gate_proj / up_proj / down_proj are the bit-exact dequantised weights."""
    from mtp_amd.repack import resolve_torch_dtype
    d, ex = store_dir
    target = resolve_torch_dtype(dtype_name)
    torch.manual_seed(0)
    with RepackedMoeExpertStore(d) as store:
        mlp = load_single_expert_mlp(store, layer=0, expert=2, bits=4, dtype=target, device="cuda")
    x = torch.randn(2, 4, mlp.hidden_size, device=mlp.gate_proj.device, dtype=mlp.gate_proj.dtype)
    with torch.inference_mode():
        out = mlp(x)
    assert bool(torch.isfinite(out).all().item())
    assert str(mlp.gate_proj.dtype).replace("torch.", "") == str(target).replace("torch.", "")
    assert list(mlp.gate_proj.shape) == [I, H] and list(mlp.up_proj.shape) == [I, H]
    assert list(mlp.down_proj.shape) == [H, I]
    assert out.shape == x.shape and out.dtype == target
    for proj, st in (("gate_proj", ex.gate), ("up_proj", ex.up), ("down_proj", ex.down)):
        want = gptq_ref.dequant_f32(st.qweight[2].numpy(), st.qzeros[2].numpy(), f16_bits(st.scales[2]))
        got = getattr(mlp, proj).float().cpu().numpy()
        # (q - z) * s is exact in fp32; the module's dtype rounds it once (RNE)
        want_t = torch.from_numpy(want).to(target).float().numpy()
        assert np.array_equal(got, want_t), proj
    xb = x.reshape(8, H).to(torch.bfloat16)
    ref = moe_ref.moe_layer_f32(bf16_bits(xb), np.full((8, 1), 2, np.int32),
                                np.ones((8, 1), np.float32), experts_to_np(ex))
    err = moe_ref.rel_err(out.reshape(8, H).float().cpu().numpy(), ref)
    print(f"  {dtype_name}: rel_err={err:.3e}", flush=True)
    assert err <= LAYER_RTOL


def test_dequantize_host_tensors_on_the_gpu(store_dir):
    """dequantize_gptq_projection given host tensors dequantises on the ROCm device and returns
    the result on the host, bit-exact."""
    from mtp_amd.repack import load_repacked_projection_tensors, dequantize_gptq_projection
    d, ex = store_dir
    with RepackedMoeExpertStore(d) as store:
        t = load_repacked_projection_tensors(store, layer=0, expert=1, projection="gate_proj")
    out = dequantize_gptq_projection(t, dtype="fp16", linear_weight=False)
    assert out.device.type == "cpu" and out.dtype == torch.float16 and out.shape == (H, I)
    want = gptq_ref.dequant_f32(ex.gate.qweight[1].numpy(), ex.gate.qzeros[1].numpy(),
                                f16_bits(ex.gate.scales[1]), linear_weight=False)
    assert np.array_equal(out.numpy(), want.astype(np.float16))


@pytest.mark.parametrize("dtype_name,mode", [("bf16", "softmax"), ("fp16", "raw")])
def test_trace_harness_call_sequence(store_dir, tmp_path, dtype_name, mode):
    """The call sequence of the reference's trace smoke harness
    (scripts/smoke_trace_topk_expert_mlp.py:60-137) on a synthetic trace sample: resolve the
    sample through a manifest, load the payload, select one token's router top-k and weights,
    load those experts, take the token's hidden state ([1, 1, H]) as input, and run the module
    with long ids and weights in the harness dtype. The output is checked against the oracle."""
    import json

    from mtp_amd.repack import resolve_torch_dtype
    from mtp_amd.tracing import (load_trace_payload, resolve_trace_sample, select_router_topk,
                                 select_trace_hidden_token)
    d, ex = store_dir
    target = resolve_torch_dtype(dtype_name)
    g = torch.Generator().manual_seed(33)
    ids = torch.stack([torch.randperm(E, generator=g)[:4] for _ in range(3)]).view(1, 3, 4)
    payload = {"router_topk": {"model.layers.0.mlp.gate": [ids]},
               "router_scores": {"model.layers.0.mlp.gate": [torch.rand(1, 3, 4, generator=g)]},
               "last_hidden_state": torch.randn(1, 3, H, generator=g)}
    (tmp_path / "s").mkdir()
    torch.save(payload, tmp_path / "s" / "sample.pt")
    (tmp_path / "manifest.jsonl").write_text(json.dumps({"path": "s/sample.pt"}) + "\n")
    sample = resolve_trace_sample(manifest_path=tmp_path / "manifest.jsonl")
    p = load_trace_payload(sample)
    sel = select_router_topk(p, layer=0, token_index=1, scores_to_weights=mode)
    with RepackedMoeExpertStore(d) as store:
        mlp = load_topk_expert_mlp(store, layer=0,
                                   expert_ids=[int(v) for v in sel.expert_ids.tolist()], bits=4,
                                   dtype=target, device="cuda")
    x = select_trace_hidden_token(p, token_index=1).to(device="cuda", dtype=target)
    w = sel.expert_weights.to(device=x.device, dtype=target)
    with torch.inference_mode():
        out = mlp(x, sel.expert_ids.to(torch.long), w)
    assert out.shape == (1, 1, H) and out.dtype == target
    assert bool(torch.isfinite(out).all().item())
    xb = x.reshape(1, H).to(torch.bfloat16)
    ref = moe_ref.moe_layer_f32(bf16_bits(xb), sel.expert_ids.numpy().astype(np.int32)[None],
                                w.float().cpu().numpy()[None], experts_to_np(ex))
    err = moe_ref.rel_err(out.reshape(1, H).float().cpu().numpy(), ref)
    print(f"  trace {dtype_name}/{mode}: rel_err={err:.3e}", flush=True)
    assert err <= LAYER_RTOL


@pytest.mark.parametrize("dtype_name", ["bf16", "fp32"])
def test_harness_call_sequences_on_the_reference_default_device(store_dir, dtype_name):
    """The reference's harnesses run with --device cpu by default (smoke_topk_expert_mlp.py:58,
    smoke_single_expert_mlp.py:36) and its loaders default to device="cpu"
    (gptq_unpack.py:337, 357): the modules then hold host tensors, the device probe finds the
    CPU, inputs are drawn there, and the outputs come back there. The kernels run on the GPU
    (host tensors staged); the results equal the oracle's and the GPU-resident module's bits."""
    from mtp_amd.repack import resolve_torch_dtype
    d, ex = store_dir
    target = resolve_torch_dtype(dtype_name)
    expert_ids = [4, 0, 7, 4]
    torch.manual_seed(1)
    with RepackedMoeExpertStore(d) as store:
        mlp = load_topk_expert_mlp(store, layer=0, expert_ids=expert_ids, bits=4, dtype=target)
        single = load_single_expert_mlp(store, layer=0, expert=2, bits=4, dtype=target)
    device = next(mlp.parameters(), next(mlp.buffers())).device
    assert device.type == "cpu"
    x = torch.randn(2, 3, mlp.hidden_size, device=device, dtype=target)
    ids = torch.tensor(expert_ids, dtype=torch.long)
    weights = torch.tensor([0.4, 0.3, 0.2, 0.1], dtype=target, device=device)
    with torch.inference_mode():
        out = mlp(x, ids, weights)
    assert out.device.type == "cpu" and out.shape == x.shape and out.dtype == target
    xb = x.reshape(6, H).to(torch.bfloat16)
    ref = moe_ref.moe_layer_f32(bf16_bits(xb), np.tile(np.array(expert_ids, np.int32), (6, 1)),
                                np.tile(weights.float().numpy(), (6, 1)), experts_to_np(ex))
    err = moe_ref.rel_err(out.reshape(6, H).float().numpy(), ref)
    print(f"  host top-k {dtype_name}: rel_err={err:.3e}", flush=True)
    assert err <= LAYER_RTOL
    gpu_out = mlp.to("cuda")(x.cuda(), ids, weights.cuda())
    assert torch.equal(gpu_out.cpu(), out)
    # single expert: inputs on mlp.gate_proj.device (the host), dense views bit-exact there
    assert single.gate_proj.device.type == "cpu" and single.gate_proj.dtype == target
    xs = torch.randn(2, 4, single.hidden_size, device=single.gate_proj.device,
                     dtype=single.gate_proj.dtype)
    with torch.inference_mode():
        ys = single(xs)
    assert ys.device.type == "cpu" and ys.shape == xs.shape
    want = gptq_ref.dequant_f32(ex.gate.qweight[2].numpy(), ex.gate.qzeros[2].numpy(),
                                f16_bits(ex.gate.scales[2]))
    assert np.array_equal(single.gate_proj.float().numpy(),
                          torch.from_numpy(want).to(target).float().numpy())
    xb = xs.reshape(8, H).to(torch.bfloat16)
    ref = moe_ref.moe_layer_f32(bf16_bits(xb), np.full((8, 1), 2, np.int32),
                                np.ones((8, 1), np.float32), experts_to_np(ex))
    assert moe_ref.rel_err(ys.reshape(8, H).float().numpy(), ref) <= LAYER_RTOL
