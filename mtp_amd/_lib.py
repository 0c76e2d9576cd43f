"""ctypes binding of libmoe_w4a16.so (the C ABI declared in include/moe_w4a16.h).

Mirrors the reference's native-library binding style: ``ctypes.CDLL`` with explicit
argtypes/restype, integer return codes turned into Python exceptions
(src/mtp_expert_prefetch/tracing/vllm_router_trace.py:8383-8445).

There is no fallback: if the library is missing the import of an op raises.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_float, POINTER, c_char_p, c_int32, c_int64, c_void_p
from pathlib import Path

LIB_NAME = "libmoe_w4a16.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME
ABI_VERSION = 2

MOE_OK = 0
MOE_ERR_NULL = 101
MOE_ERR_SHAPE = 102
MOE_ERR_UNSUPPORTED = 103
MOE_ERR_WORKSPACE = 104
MOE_ERR_HIP = 200

PATH_AUTO = 0
PATH_DECODE = 1
PATH_PREFILL = 2

EXPORTED = (
    "moe_w4a16_abi_version",
    "moe_w4a16_last_error",
    "moe_dequant_v1",
    "moe_router_topk_v1",
    "moe_capacity_blocks_v1",
    "moe_align_v1",
    "moe_w1_gateup_silu_v1",
    "moe_w2_down_v1",
    "moe_sum_v1",
    "moe_rmsnorm_v1",
    "moe_layer_workspace_bytes_v1",
    "moe_layer_v1",
    "moe_norm_layer_v1",
    "moe_fused_experts_v1",
    "moe_layer_noalloc_max_bytes_v1",
    "moe_layer_noalloc_v1",
    "moe_predictor_workspace_bytes_v1",
    "moe_predictor_v1",
    "moe_awq_to_gptq_v1",
    "moe_hr_predictor_workspace_bytes_v1",
    "moe_hr_predictor_v1",
    "moe_slot_cache_create_v1",
    "moe_slot_cache_destroy_v1",
    "moe_slot_cache_prefetch_v1",
    "moe_slot_cache_demand_v1",
    "moe_slot_cache_layer_done_v1",
    "moe_slot_cache_stats_v1",
    "moe_slot_cache_slot_of_v1",
    "moe_offload_layer_v1",
    "moe_ready_cache_create_v1",
    "moe_ready_cache_destroy_v1",
    "moe_ready_cache_prefetch_v1",
    "moe_ready_cache_demand_v1",
    "moe_ready_cache_advance_v1",
    "moe_ready_cache_finish_v1",
    "moe_ready_cache_stats_v1",
)


class SlotCacheDesc(ctypes.Structure):
    _fields_ = [
        ("num_layers", c_int32),
        ("num_experts", c_int32),
        ("slots_per_layer", c_int32),
        ("device", c_int32),
        ("expert_bytes", c_int64),
        ("host_pool", c_void_p),
        ("device_pool", c_void_p),
        ("device_expert_row", c_void_p),
        ("dry_run", c_int32),
        ("ready_deadline_us", c_float),
    ]


class SlotCacheCounters(ctypes.Structure):
    _fields_ = [(name, c_int64) for name in (
        "capacity", "resident_count", "issued_fetch_count", "used_fetch_count",
        "unused_fetch_count", "demand_count", "demand_hit_count", "demand_miss_count",
        "evicted_before_use_count", "prefetch_bytes", "demand_bytes",
        "prefetch_skipped_pinned_count", "ready_late_miss_count", "ready_late_wait_ns")]


class ReadyCacheStats(ctypes.Structure):
    _fields_ = [(name, c_int64) for name in (
        "capacity", "resident_count", "issued_fetch_count", "used_fetch_count",
        "unused_fetch_count", "demand_count", "demand_hit_count", "demand_miss_count",
        "evicted_before_use_count", "ready_late_miss_count", "late_completion_unused_count",
        "queue_batch_count")] + [(name, ctypes.c_double) for name in (
        "queue_service_us", "queue_total_span_us", "queue_wait_us", "queue_max_delay_us",
        "queue_event_interval_us", "queue_deadline_us")] + [("queue_batch_size", c_int64)]


class HrPredictorParams(ctypes.Structure):
    _fields_ = [(name, c_void_p) for name in (
        "enc_w", "enc_b", "ln_w", "ln_b", "layer_emb", "delta_emb", "cls_w", "cls_b")] + [
        (name, c_int32) for name in ("hidden", "width", "num_layers", "future_window",
                                     "num_experts")] + [("ln_eps", c_float)]


class GptqProj(ctypes.Structure):
    _fields_ = [("qweight", c_void_p), ("qzeros", c_void_p), ("scales", c_void_p)]


class ExpertSet(ctypes.Structure):
    _fields_ = [
        ("gate", GptqProj),
        ("up", GptqProj),
        ("down", GptqProj),
        ("expert_row", c_void_p),
        ("num_experts", c_int32),
        ("hidden", c_int32),
        ("intermediate", c_int32),
        ("group_size", c_int32),
        ("expert_stride_bytes", c_int64),
    ]


class MoeLibraryError(RuntimeError):
    def __init__(self, code: int, message: str) -> None:
        super().__init__(f"[moe_w4a16 error {code}] {message}")
        self.code = code


_LIB: ctypes.CDLL | None = None

_P = c_void_p
_I = c_int32
_SIGS = {
    "moe_w4a16_abi_version": ([], c_int32),
    "moe_w4a16_last_error": ([], c_char_p),
    "moe_dequant_v1": ([POINTER(GptqProj), _P, _I, _I, _I, _I, _I, _I, _P, _P], c_int32),
    "moe_router_topk_v1": ([_P, _I, _I, _P, _I, _P, _I, _P, _P, _P, _P, _P], c_int32),
    "moe_capacity_blocks_v1": ([_I, _I, _I, _I, _I], c_int32),
    "moe_align_v1": ([_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P], c_int32),
    "moe_w1_gateup_silu_v1": (
        [_P, _I, _I, POINTER(ExpertSet), POINTER(ExpertSet), _P, _P, _P, _I, _I, _P, _I, _P],
        c_int32),
    "moe_w2_down_v1": (
        [_P, _I, _I, POINTER(ExpertSet), POINTER(ExpertSet), _P, _P, _P, _I, _I, _P, _P, _I, _P],
        c_int32),
    "moe_sum_v1": ([_P, _I, _I, _I, _I, _P, _I, _P, _P, _P], c_int32),
    "moe_rmsnorm_v1": ([_P, _P, _I, _I, _P, c_float, _P, _P], c_int32),
    "moe_layer_workspace_bytes_v1": ([_I, _I, POINTER(ExpertSet), _I, _I], c_int64),
    "moe_layer_v1": (
        [_P, _I, _P, _P, _I, POINTER(ExpertSet), POINTER(ExpertSet), _P, _P, c_int64, _P, _P, _P,
         _I, _P],
        c_int32),
    "moe_norm_layer_v1": (
        [_P, _P, _P, c_float, _P, _P, _I, _P, _P, _I, POINTER(ExpertSet), POINTER(ExpertSet), _P,
         _P, c_int64, _P, _P, _P, _I, _P],
        c_int32),
    "moe_layer_noalloc_max_bytes_v1": ([], c_int64),
    "moe_layer_noalloc_v1": (
        [_P, _I, _P, _P, _I, POINTER(ExpertSet), POINTER(ExpertSet), _P, _P, _P, _P, _I, _P],
        c_int32),
    "moe_fused_experts_v1": (
        [_P, _I, _P, _P, _I, POINTER(ExpertSet), POINTER(ExpertSet), _P, _P, c_int64, _P, _I, _P],
        c_int32),
    "moe_predictor_workspace_bytes_v1": ([_I, _I, _I, _I, _I], c_int64),
    "moe_predictor_v1": ([_P, _I, _I, _I, _P, _I, _P, _I, _I, _P, c_int64, _P, _P], c_int32),
    "moe_awq_to_gptq_v1": ([_I, _P, _P, _P, _I, _I, _I, _I, _I, POINTER(GptqProj), _P, _P], c_int32),
    "moe_hr_predictor_workspace_bytes_v1": ([_I, POINTER(HrPredictorParams)], c_int64),
    "moe_hr_predictor_v1": ([_P, _I, _P, POINTER(HrPredictorParams), _P, c_float, _P, _I, _P, c_int64,
                             _P, _P, _P], c_int32),
    "moe_slot_cache_create_v1": ([POINTER(SlotCacheDesc), POINTER(ctypes.c_uint64)], c_int32),
    "moe_slot_cache_destroy_v1": ([ctypes.c_uint64], c_int32),
    "moe_slot_cache_prefetch_v1": ([ctypes.c_uint64, _I, _P, _I, _P, POINTER(c_int32)], c_int32),
    "moe_slot_cache_demand_v1": ([ctypes.c_uint64, _I, _P, _I, _P, POINTER(c_int32)], c_int32),
    "moe_slot_cache_layer_done_v1": ([ctypes.c_uint64, _I], c_int32),
    "moe_slot_cache_stats_v1": ([ctypes.c_uint64, POINTER(SlotCacheCounters)], c_int32),
    "moe_slot_cache_slot_of_v1": ([ctypes.c_uint64, _I, _I], c_int32),
    "moe_offload_layer_v1": (
        [ctypes.c_uint64, _I, _P, _I, _P, _P, _I, POINTER(ExpertSet), _P, c_int64, _P, _P, _P, _I,
         _I, _P, POINTER(c_int32)],
        c_int32),
    "moe_ready_cache_create_v1": ([_I, c_int64, ctypes.c_double, ctypes.c_double, c_int64,
                                   ctypes.c_double, POINTER(ctypes.c_uint64)], c_int32),
    "moe_ready_cache_destroy_v1": ([ctypes.c_uint64], c_int32),
    "moe_ready_cache_prefetch_v1": ([ctypes.c_uint64, _I, _P, _I, ctypes.c_double, _P,
                                     POINTER(c_int32)], c_int32),
    "moe_ready_cache_demand_v1": ([ctypes.c_uint64, _I, _P, _I, ctypes.c_double, _P,
                                   POINTER(c_int32)], c_int32),
    "moe_ready_cache_advance_v1": ([ctypes.c_uint64, ctypes.c_double], c_int32),
    "moe_ready_cache_finish_v1": ([ctypes.c_uint64], c_int32),
    "moe_ready_cache_stats_v1": ([ctypes.c_uint64, POINTER(ReadyCacheStats)], c_int32),
}


def lib_path() -> Path:
    override = os.environ.get("MTP_AMD_LIB")
    return Path(override) if override else LIB_PATH


def load() -> ctypes.CDLL:
    """Load the library once; raise if it is missing or its ABI does not match."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = lib_path()
    if not path.exists():
        raise RuntimeError(
            f"{path} is missing: the MI355X kernels are not built. "
            "Run `python -m mtp_amd.build` (or __graft_entry__.build()) first; there is no CPU fallback."
        )
    lib = ctypes.CDLL(str(path))
    for name, (argtypes, restype) in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    version = lib.moe_w4a16_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {version}, expected {ABI_VERSION}")
    _LIB = lib
    return lib


def check(code: int) -> None:
    if code != MOE_OK:
        msg = load().moe_w4a16_last_error().decode("utf-8", "replace")
        raise MoeLibraryError(code, msg)
