"""moe_layer_noalloc_v1 (the layer with its workspace in a file-scope device array, no
allocation) against moe_layer_v1 with a caller workspace, through the C ABI: outputs and routing
bit-identical on two calls in a row, the second smaller, and an oversized call refused."""

from __future__ import annotations

import ctypes

import pytest
import torch

from mtp_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu


def _noalloc(lib, x, layer, top_k, path, shared=False):
    T = x.shape[0]
    out = torch.full_like(x, float("nan"))
    ids = torch.full((T, top_k), -7, dtype=torch.int32, device=x.device)
    w = torch.full((T, top_k), float("nan"), dtype=torch.float32, device=x.device)
    ex = layer.experts.struct()
    sh = layer.shared.struct() if shared else None
    rc = lib.moe_layer_noalloc_v1(
        x.data_ptr(), T, layer.router_w.data_ptr(),
        None if layer.logit_bias is None else layer.logit_bias.data_ptr(), top_k,
        ctypes.byref(ex), ctypes.byref(sh) if sh else None,
        layer.shared_gate_w.data_ptr() if shared else None, out.data_ptr(), ids.data_ptr(),
        w.data_ptr(), ops.PATHS[path], ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return rc, out, ids, w


def _reference(x, layer, top_k, path, shared=False):
    return ops.moe_layer(x, layer.router_w, layer.experts, top_k=top_k, logit_bias=layer.logit_bias,
                         shared=layer.shared if shared else None,
                         shared_gate_w=layer.shared_gate_w if shared else None, path=path,
                         return_routing=True)


def test_noalloc_layer_matches_workspace_layer_on_consecutive_calls():
    lib = _lib.load()
    assert lib.moe_layer_noalloc_max_bytes_v1() == 64 << 20
    layer = synth.layer_to(synth.make_layer(11, zipf=True, shared=True), "cuda")
    # the second call is smaller and takes another path: the scratch keeps the first call's
    # bytes, which the layer must not depend on
    for T, path, shared in ((384, "auto", True), (5, "decode", False)):
        print(f"noalloc T={T} path={path} shared={shared}", flush=True)
        x = synth.make_tokens(T, seed=300 + T).cuda()
        rc, out, ids, w = _noalloc(lib, x, layer, 8, path, shared)
        torch.cuda.synchronize()
        _lib.check(rc)
        ref_out, ref_ids, ref_w = _reference(x, layer, 8, path, shared)
        torch.cuda.synchronize()
        assert torch.equal(ids, ref_ids)
        assert torch.equal(w, ref_w)
        assert torch.equal(out, ref_out)


def test_noalloc_layer_refuses_calls_beyond_its_scratch():
    lib = _lib.load()
    layer = synth.layer_to(synth.make_layer(12), "cuda")
    x = synth.make_tokens(1024, seed=5).cuda()
    need = ops.workspace_bytes(1024, 8, layer.experts, False, "auto")
    assert need > lib.moe_layer_noalloc_max_bytes_v1()
    rc, out, _, _ = _noalloc(lib, x, layer, 8, "auto")
    torch.cuda.synchronize()
    assert rc == _lib.MOE_ERR_WORKSPACE
    assert b"scratch" in lib.moe_w4a16_last_error()
    assert bool(torch.isnan(out.float()).all())  # nothing was launched
