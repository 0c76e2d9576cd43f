"""C-ABI checks that need no GPU: the library loads, exports every symbol the header declares,
and its host-side validation returns the documented error codes (no kernel is launched)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from mtp_amd import _lib, ops
from oracle import moe_ref

HEADER = Path(__file__).resolve().parents[1] / "include" / "moe_w4a16.h"


def header_functions() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^(?:int|int64_t|const char\*)\s+(moe_[a-z0-9_]+)\(", text, flags=re.M)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = header_functions()
    assert declared, "no declarations parsed from the header"
    assert sorted(declared) == sorted(_lib.EXPORTED)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.moe_w4a16_abi_version() == _lib.ABI_VERSION


def _fake_set(E=256, H=2048, I=512, G=128) -> _lib.ExpertSet:
    p = _lib.GptqProj(0x1000, 0x2000, 0x3000)  # never dereferenced by the host-side checks
    return _lib.ExpertSet(p, p, p, None, E, H, I, G)


def test_null_and_shape_errors_are_reported():
    lib = _lib.load()
    rc = lib.moe_layer_v1(None, 4, None, None, 8, None, None, None, None, 0, None, None, None, 0, None)
    assert rc == _lib.MOE_ERR_NULL
    assert b"experts is NULL" in lib.moe_w4a16_last_error()
    bad = _fake_set(H=1000)
    rc = lib.moe_w1_gateup_silu_v1(None, 4, 8, ctypes.byref(bad), None, None, None, None, 16, 1,
                                   None, 0, None)
    assert rc == _lib.MOE_ERR_SHAPE
    with pytest.raises(_lib.MoeLibraryError) as err:
        _lib.check(rc)
    assert err.value.code == _lib.MOE_ERR_SHAPE and "hidden=1000" in str(err.value)
    rc = lib.moe_router_topk_v1(0x10, 1, 2048, 0x10, 256, None, 300, None, 0x10, 0x10, 0x10, None)
    assert rc == _lib.MOE_ERR_SHAPE
    rc = lib.moe_align_v1(0x10, 4, 8, 256, 0, 16, 1, 0x10, 0x10, 0x10, None)
    assert rc == _lib.MOE_ERR_WORKSPACE


def test_workspace_too_small_is_rejected():
    lib = _lib.load()
    ex = _fake_set()
    need = lib.moe_layer_workspace_bytes_v1(16, 8, ctypes.byref(ex), 0, 0)
    assert need > 0
    rc = lib.moe_layer_v1(0x10, 16, 0x10, None, 8, ctypes.byref(ex), None, None, 0x10, need - 1,
                          0x10, None, None, 0, None)
    assert rc == _lib.MOE_ERR_WORKSPACE


@pytest.mark.parametrize("base", [0x1004, 0x1080])
def test_misaligned_workspace_is_rejected_before_any_launch(base):
    """Workspaces start on 256-byte boundaries; an entry point refuses another base up front."""
    lib = _lib.load()
    ex = _fake_set()
    need = lib.moe_layer_workspace_bytes_v1(16, 8, ctypes.byref(ex), 0, 0)
    rc = lib.moe_layer_v1(0x10, 16, 0x10, None, 8, ctypes.byref(ex), None, None, base, need,
                          0x10, None, None, 0, None)
    assert rc == _lib.MOE_ERR_WORKSPACE
    assert b"256-byte aligned" in lib.moe_w4a16_last_error()
    rc = lib.moe_fused_experts_v1(0x10, 16, 0x10, 0x10, 8, ctypes.byref(ex), None, None, base,
                                  need, 0x10, 0, None)
    assert rc == _lib.MOE_ERR_WORKSPACE


@pytest.mark.parametrize("path", [3, -1, 99])
def test_unknown_path_is_refused(path):
    """Only AUTO, DECODE and PREFILL exist; any other path value is an error, never AUTO."""
    lib = _lib.load()
    ex = _fake_set()
    assert lib.moe_layer_workspace_bytes_v1(16, 8, ctypes.byref(ex), 0, path) == -1
    need = lib.moe_layer_workspace_bytes_v1(16, 8, ctypes.byref(ex), 0, 0)
    rc = lib.moe_layer_v1(0x10, 16, 0x10, None, 8, ctypes.byref(ex), None, None, 0x10, need,
                          0x10, None, None, path, None)
    assert rc == _lib.MOE_ERR_UNSUPPORTED
    assert f"unknown path {path}".encode() in lib.moe_w4a16_last_error()
    rc = lib.moe_w1_gateup_silu_v1(0x10, 4, 8, ctypes.byref(ex), None, 0x10, 0x10, 0x10, 16, 1,
                                   0x10, path, None)
    assert rc == _lib.MOE_ERR_UNSUPPORTED


@pytest.mark.parametrize("T,k,E,shared,BM", [(1, 8, 256, 0, 16), (64, 8, 256, 1, 16),
                                               (2048, 8, 256, 0, 128), (3, 4, 16, 1, 4)])
def test_capacity_blocks_matches_oracle_bound(T, k, E, shared, BM):
    lib = _lib.load()
    got = lib.moe_capacity_blocks_v1(T, k, E, shared, BM)
    assert got == moe_ref.max_blocks(T * k + (T if shared else 0), E + shared, BM)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setenv("MTP_AMD_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.load()


def test_predictor_rejects_weights_beyond_32_bit_offsets():
    """The predictor's GEMV kernels use 32-bit buffer offsets: heads whose bf16 weights reach
    2 GiB are refused before any launch (here 40 heads of 8192 x 4096 = 2.5 GiB of w1)."""
    lib = _lib.load()
    ws_need = lib.moe_predictor_workspace_bytes_v1(1, 40, 8192, 256, 16)
    rc = lib.moe_predictor_v1(0x10, 1, 4096, 40, 0x10, 8192, 0x10, 256, 16, 0x10, ws_need, 0x10,
                              None)
    assert rc == _lib.MOE_ERR_SHAPE
    assert b"exceed 2 GiB" in lib.moe_w4a16_last_error()
    # the full-size workload shape (40 heads of 1024 x 2048) is accepted by the checks
    ws_need = lib.moe_predictor_workspace_bytes_v1(1, 40, 1024, 256, 16)
    assert ws_need > 0


def test_moe_sum_requires_the_routed_ids():
    lib = _lib.load()
    rc = lib.moe_sum_v1(0x10, 4, 8, 2048, 0, None, 256, None, 0x10, None)
    assert rc == _lib.MOE_ERR_NULL


@pytest.mark.parametrize("T,top_k,path,E", [(16, 8, 3, 256), (16, 8, -1, 256), (16, 65, 0, 256),
                                            (4, 20, 1, 16), (4, 0, 0, 256), (-1, 8, 0, 256)])
def test_noalloc_entry_reports_the_workspace_entrys_error_codes(T, top_k, path, E):
    """moe_layer_noalloc_v1 runs moe_layer_v1's argument checks before its scratch-size check:
    an unknown path, a top_k outside [1, min(E, 64)] or a negative T get the same code and
    message from both entry points (checked on the host; nothing is launched)."""
    lib = _lib.load()
    ex = _fake_set(E=E)
    rc_ws = lib.moe_layer_v1(0x10, T, 0x10, None, top_k, ctypes.byref(ex), None, None, 0x10,
                             1 << 40, 0x10, None, None, path, None)
    msg_ws = lib.moe_w4a16_last_error()
    rc_na = lib.moe_layer_noalloc_v1(0x10, T, 0x10, None, top_k, ctypes.byref(ex), None, None,
                                     0x10, None, None, path, None)
    assert rc_ws != _lib.MOE_OK
    assert rc_na == rc_ws
    assert lib.moe_w4a16_last_error() == msg_ws


@pytest.mark.parametrize("T,k", [(1, 8), (255, 8), (319, 8), (320, 8), (2048, 8), (2559, 1),
                                 (2560, 1), (40, 64)])
def test_auto_path_switches_at_the_measured_slot_count(T, k):
    """AUTO runs the decode kernels below 2 560 routed slots and the prefill kernels from there
    on (the two paths' workspaces differ in their block tables, so the query shows which)."""
    lib = _lib.load()
    ex = _fake_set()
    sizes = {p: lib.moe_layer_workspace_bytes_v1(T, k, ctypes.byref(ex), 0, p)
             for p in (_lib.PATH_AUTO, _lib.PATH_DECODE, _lib.PATH_PREFILL)}
    assert sizes[_lib.PATH_DECODE] != sizes[_lib.PATH_PREFILL]
    want = _lib.PATH_PREFILL if T * k >= 2560 else _lib.PATH_DECODE
    assert sizes[_lib.PATH_AUTO] == sizes[want]
    assert ops._block_m(_lib.PATH_AUTO, T, k) == (128 if want == _lib.PATH_PREFILL else 16)
