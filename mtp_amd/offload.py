"""Offloaded experts: every (layer, expert) blob in pinned host memory, an HBM slot pool per layer,
prefetch on a side stream driven by a predictor, demand fetch of misses on the compute stream.

Reference behaviour this replaces:
  * cache accounting  src/mtp_expert_prefetch/runtime/cache_manager.py:208-279
    (ControlledExpertCacheManager: LRU per (layer, expert), counters issued / used / unused /
    evicted-before-use / demand hit / miss). Here the capacity is per layer (the slots of that
    layer's HBM pool) and the bytes really move (hipMemcpyAsync H2D).
  * predictor         src/mtp_expert_prefetch/training/hidden_residual.py:44-106, simplified to
    one bf16 MLP head per layer (hidden -> inner SiLU -> experts) whose top-k is prefetched.

Expert blob: the nine GPTQ tensors of one expert back to back (no g_idx; the kernels assume
g_idx[k] = k // group_size), in the order gate, up, down and qweight, qzeros, scales inside each
projection. At the Qwen3-MoE shape (H 2048, I 512, G 128) the blob is 1 634 304 bytes. The
kernels read a layer's slots through an ExpertSet whose tensors point into slot 0 of that layer
with expert_stride_bytes = blob size and expert_row = the layer's expert -> slot table.
"""

from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass

import torch

from mtp_amd import _lib, ops
from mtp_amd.weights import GptqStack, MoeExperts

PIECES = ("qweight", "qzeros", "scales")
PROJ_ORDER = ("gate", "up", "down")


@dataclass(frozen=True)
class BlobPiece:
    proj: str
    kind: str
    offset: int
    shape: tuple[int, int]
    dtype: torch.dtype

    @property
    def nbytes(self) -> int:
        return self.shape[0] * self.shape[1] * torch.empty((), dtype=self.dtype).element_size()


def blob_layout(hidden: int, inter: int, group_size: int) -> tuple[list[BlobPiece], int]:
    """Pieces of one expert blob (offsets in bytes) and the blob size."""
    pieces: list[BlobPiece] = []
    off = 0
    for proj, (k, n) in zip(PROJ_ORDER, ((hidden, inter), (hidden, inter), (inter, hidden))):
        if k % group_size or k % 8 or n % 8:
            raise ValueError(f"{proj}: in={k} out={n} group={group_size} do not tile")
        for kind, shape, dtype in (("qweight", (k // 8, n), torch.int32),
                                   ("qzeros", (k // group_size, n // 8), torch.int32),
                                   ("scales", (k // group_size, n), torch.float16)):
            piece = BlobPiece(proj, kind, off, shape, dtype)
            if off % 16:
                raise ValueError("blob pieces must stay 16-byte aligned")
            pieces.append(piece)
            off += piece.nbytes
    if off % 16:
        raise ValueError("blob size must be a multiple of 16 bytes")
    return pieces, off


def pack_blobs(experts: MoeExperts) -> torch.Tensor:
    """uint8 [num_experts, blob] of a resident (contiguous) expert set, on its device."""
    experts.validate()
    pieces, _ = blob_layout(experts.hidden_size, experts.intermediate_size, experts.group_size)
    stacks = {"gate": experts.gate, "up": experts.up, "down": experts.down}
    parts = []
    for p in pieces:
        t = getattr(stacks[p.proj], p.kind)
        parts.append(t.reshape(t.shape[0], -1).view(torch.uint8))
    return torch.cat(parts, dim=1)


# ----------------------------------------------------------------------------- pinned host memory
class PinnedHostBuffer:
    """hipHostMalloc'd host memory (page-locked, so hipMemcpyAsync from it is a true async DMA).

    Allocated through the HIP runtime that torch has already loaded (one runtime per process).
    """

    def __init__(self, nbytes: int) -> None:
        if nbytes <= 0:
            raise ValueError("nbytes must be positive")
        torch.cuda.init()
        self._hip = ctypes.CDLL("libamdhip64.so.7")
        self._hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t,
                                            ctypes.c_uint]
        self._hip.hipHostMalloc.restype = ctypes.c_int
        self._hip.hipHostFree.argtypes = [ctypes.c_void_p]
        self._hip.hipHostFree.restype = ctypes.c_int
        ptr = ctypes.c_void_p()
        err = self._hip.hipHostMalloc(ctypes.byref(ptr), ctypes.c_size_t(nbytes), 0)
        if err != 0 or not ptr.value:
            raise MemoryError(f"hipHostMalloc({nbytes}) failed with HIP error {err}")
        self.ptr = int(ptr.value)
        self.nbytes = int(nbytes)

    def view(self) -> torch.Tensor:
        """A CPU uint8 tensor over the buffer (valid while the buffer is open)."""
        if not self.ptr:
            raise RuntimeError("buffer is closed")
        arr = (ctypes.c_uint8 * self.nbytes).from_address(self.ptr)
        return torch.frombuffer(arr, dtype=torch.uint8)

    def close(self) -> None:
        if self.ptr:
            self._hip.hipHostFree(ctypes.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self) -> None:  # pragma: no cover - interpreter teardown order varies
        try:
            self.close()
        except Exception:
            pass


# ----------------------------------------------------------------------------- slot cache
class SlotCache:
    """ctypes handle of moe_slot_cache_*_v1. dry_run=True keeps only the accounting."""

    def __init__(self, num_layers: int, num_experts: int, slots_per_layer: int, expert_bytes: int,
                 *, host_pool: int = 0, device_pool: int = 0, expert_row: int = 0,
                 device: int = 0, dry_run: bool = False, ready_deadline_us: float = 0.0) -> None:
        self._lib = _lib.load()
        desc = _lib.SlotCacheDesc(num_layers, num_experts, slots_per_layer, device, expert_bytes,
                                  host_pool, device_pool, expert_row, int(dry_run),
                                  float(ready_deadline_us))
        handle = ctypes.c_uint64()
        _lib.check(self._lib.moe_slot_cache_create_v1(ctypes.byref(desc), ctypes.byref(handle)))
        self.handle = handle.value
        self.num_layers = num_layers
        self.num_experts = num_experts
        self.dry_run = dry_run

    @staticmethod
    def _ids(experts) -> tuple[ctypes.Array, int]:
        vals = [int(e) for e in experts]
        return (ctypes.c_int32 * max(len(vals), 1))(*vals), len(vals)

    def _stream(self, stream) -> int | None:
        if self.dry_run:
            return None
        s = stream if stream is not None else torch.cuda.current_stream()
        return s.cuda_stream

    def prefetch(self, layer: int, experts, stream=None) -> int:
        """Start copies of the non-resident experts on the side stream; returns copies started."""
        arr, n = self._ids(experts)
        issued = ctypes.c_int32()
        _lib.check(self._lib.moe_slot_cache_prefetch_v1(self.handle, layer, arr, n,
                                                        self._stream(stream), ctypes.byref(issued)))
        return issued.value

    def demand(self, layer: int, experts, stream=None) -> int:
        """Make the experts resident before the next work on `stream`; returns hits."""
        arr, n = self._ids(experts)
        hits = ctypes.c_int32()
        _lib.check(self._lib.moe_slot_cache_demand_v1(self.handle, layer, arr, n,
                                                      self._stream(stream), ctypes.byref(hits)))
        return hits.value

    def layer_done(self, layer: int) -> None:
        """The kernels reading the layer's slots (after its latest demand) are enqueued: its
        slots may be taken by prefetches again."""
        _lib.check(self._lib.moe_slot_cache_layer_done_v1(self.handle, layer))

    def stats(self) -> dict[str, int]:
        c = _lib.SlotCacheCounters()
        _lib.check(self._lib.moe_slot_cache_stats_v1(self.handle, ctypes.byref(c)))
        return {name: int(getattr(c, name)) for name, _ in _lib.SlotCacheCounters._fields_}

    def slot_of(self, layer: int, expert: int) -> int:
        s = int(self._lib.moe_slot_cache_slot_of_v1(self.handle, layer, expert))
        if s == -2:
            raise IndexError(f"(layer {layer}, expert {expert}) out of range")
        return s

    def close(self) -> None:
        if self.handle:
            _lib.check(self._lib.moe_slot_cache_destroy_v1(self.handle))
            self.handle = 0

    def __enter__(self) -> "SlotCache":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


# ----------------------------------------------------------------------------- offloaded layers
class OffloadedExperts:
    """Host pool of [num_layers][num_experts] blobs, HBM pool of [num_layers][slots] blobs, and
    the slot cache that moves blobs between them.

    Fill the host pool with `store_layer`, then per layer: `demand` the routed experts, run the
    kernels on `layer_experts(layer)`, and `prefetch` predicted experts of later steps.
    """

    def __init__(self, num_layers: int, num_experts: int, hidden: int, inter: int,
                 slots_per_layer: int, *, group_size: int = 128, device=None) -> None:
        self.device = torch.device(device if device is not None else "cuda")
        if self.device.type != "cuda":
            raise ValueError("offloaded experts need a ROCm device")
        self.num_layers, self.num_experts = num_layers, num_experts
        self.hidden, self.inter, self.group_size = hidden, inter, group_size
        self.slots = slots_per_layer
        self.pieces, self.blob = blob_layout(hidden, inter, group_size)
        self.host = PinnedHostBuffer(num_layers * num_experts * self.blob)
        self.device_pool = torch.empty(num_layers, max(slots_per_layer, 1), self.blob,
                                       dtype=torch.uint8, device=self.device)
        # expert -> slot table; -1 = not resident (kernels drop such slots)
        self.expert_row = torch.full((num_layers, num_experts), -1, dtype=torch.int32,
                                     device=self.device)
        self.cache = SlotCache(num_layers, num_experts, slots_per_layer, self.blob,
                               host_pool=self.host.ptr, device_pool=self.device_pool.data_ptr(),
                               expert_row=self.expert_row.data_ptr(),
                               device=self.device.index or 0)
        self._views = [self._layer_view(l) for l in range(num_layers)]

    def _layer_view(self, layer: int) -> MoeExperts:
        base = self.device_pool[layer]  # [slots, blob] uint8
        stacks = {}
        for proj in PROJ_ORDER:
            parts = {}
            for p in self.pieces:
                if p.proj != proj:
                    continue
                width = p.nbytes // torch.empty((), dtype=p.dtype).element_size()
                v = base[:, p.offset:p.offset + p.nbytes].view(p.dtype)  # [slots, width]
                parts[p.kind] = v.as_strided((v.shape[0],) + p.shape, (v.stride(0), p.shape[1], 1))
                assert width == p.shape[0] * p.shape[1]
            stacks[proj] = GptqStack(parts["qweight"], parts["qzeros"], parts["scales"])
        return MoeExperts(stacks["gate"], stacks["up"], stacks["down"], self.group_size,
                          expert_row=self.expert_row[layer], num_experts=self.num_experts,
                          expert_stride_bytes=self.blob)

    def reset_cache(self) -> None:
        """Forget every resident slot and counter (pools are kept; the next demands refetch)."""
        torch.cuda.synchronize(self.device)
        self.cache.close()
        self.expert_row.fill_(-1)
        self.cache = SlotCache(self.num_layers, self.num_experts, self.slots, self.blob,
                               host_pool=self.host.ptr, device_pool=self.device_pool.data_ptr(),
                               expert_row=self.expert_row.data_ptr(),
                               device=self.device.index or 0)

    def layer_experts(self, layer: int) -> MoeExperts:
        """Expert set of one layer reading its HBM slots (valid after `demand`)."""
        return self._views[layer]

    def store_layer(self, layer: int, experts: MoeExperts) -> None:
        """Copy a resident layer's experts into the host pool (blob layout)."""
        if (experts.hidden_size, experts.intermediate_size, experts.group_size) != (
                self.hidden, self.inter, self.group_size):
            raise ValueError("expert shapes do not match the pool")
        if experts.gate.num_rows != self.num_experts or experts.expert_row is not None:
            raise ValueError("store_layer needs a dense stack of all num_experts experts")
        blobs = pack_blobs(experts)
        n = self.num_experts * self.blob
        dst = self.host.view()[layer * n:(layer + 1) * n]
        dst.copy_(blobs.reshape(-1))  # device -> pinned host DMA when the stack is on the GPU
        del blobs

    def load_from_store(self, store, layer: int, *, store_layer: int | None = None,
                        verify: bool = True) -> None:
        """Fill pool layer `layer` from a repacked store (store layer `store_layer`, default the
        same index): every expert's nine GPTQ tensors are copied from the layer file straight
        into its blob in pinned host memory, after the manifest checks of
        RepackedMoeExpertStore.read_layer_tensors (shape, dtype, sha256 with verify). The
        store's g_idx must be k // group_size (the layout the kernels address)."""
        src_layer = layer if store_layer is None else store_layer
        t = store.read_layer_tensors(src_layer, verify=verify)
        names = {"gate": "gate_proj", "up": "up_proj", "down": "down_proj"}
        for proj, name in names.items():
            gi = t[f"experts.{name}.g_idx"].to(torch.int64)
            k = gi.shape[-1]
            if gi.shape[0] != self.num_experts or not bool(
                    (gi == torch.arange(k) // self.group_size).all()):
                raise NotImplementedError(
                    f"layer {src_layer} {name}: g_idx must be k // {self.group_size} for every "
                    f"one of {self.num_experts} experts")
        n = self.num_experts * self.blob
        host = self.host.view()[layer * n:(layer + 1) * n].view(self.num_experts, self.blob)
        for p in self.pieces:
            src = t[f"experts.{names[p.proj]}.{p.kind}"]
            if p.kind == "scales":
                src = src.to(torch.float16)
            if tuple(src.shape) != (self.num_experts,) + p.shape or src.dtype != p.dtype:
                raise ValueError(f"layer {src_layer} {names[p.proj]}.{p.kind}: shape "
                                 f"{tuple(src.shape)} {src.dtype} does not fit the pool "
                                 f"({(self.num_experts,) + p.shape} {p.dtype})")
            host[:, p.offset:p.offset + p.nbytes].copy_(
                src.contiguous().view(torch.uint8).reshape(self.num_experts, p.nbytes))

    def prefetch(self, layer: int, experts, stream=None) -> int:
        return self.cache.prefetch(layer, experts, stream)

    def demand(self, layer: int, experts, stream=None) -> int:
        return self.cache.demand(layer, experts, stream)

    def layer_done(self, layer: int) -> None:
        self.cache.layer_done(layer)

    def stats(self) -> dict[str, int]:
        return self.cache.stats()

    def close(self) -> None:
        torch.cuda.synchronize(self.device)
        self.cache.close()
        self.expert_row.fill_(-1)
        self.host.close()


def routed_layer(x: torch.Tensor, router_w: torch.Tensor, pool: OffloadedExperts, layer: int, *,
                 top_k: int = 8, logit_bias: torch.Tensor | None = None,
                 ids_host: torch.Tensor | None = None, path: str = "auto",
                 workspace: torch.Tensor | None = None,
                 prefetch: list[int] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """One offloaded MoE layer in one native call (moe_offload_layer_v1): router -> ids to the
    host -> demand -> experts from the slots [-> prefetch of `prefetch`, the demand's slots still
    pinned] -> layer_done.

    The host wait for the routed ids is the one synchronisation per layer that a host-managed
    cache needs (the reference's demand() is a host call on the routed ids too,
    cache_manager.py:233-247). A pinned ids_host (the default) receives the ids from the top-k
    kernel itself; a pageable one gets a copy. Returns (out bf16 [T, H], routed ids on the host
    int32 [T, k]).
    """
    lib = _lib.load()
    ex = pool.layer_experts(layer)
    ops._bf16_matrix(x, "input", ex.hidden_size)
    ops._bf16_matrix(router_w, "router_w", ex.hidden_size)
    if router_w.shape[0] != ex.num_experts:
        raise ValueError(f"router_w has {router_w.shape[0]} rows for {ex.num_experts} experts")
    ops._check_bias_gate(logit_bias, None, ex.num_experts, ex.hidden_size)
    ops._require_gpu(x, router_w, logit_bias)
    T = x.shape[0]
    p = ops._path(path)
    workspace = ops._workspace(workspace, ops.workspace_bytes(T, top_k, ex, False, p), x.device)
    if ids_host is None or tuple(ids_host.shape) != (T, top_k):
        ids_host = torch.empty((T, top_k), dtype=torch.int32, pin_memory=True)
    elif (ids_host.device.type != "cpu" or ids_host.dtype != torch.int32
          or not ids_host.is_contiguous()):
        # the cache's demand reads the routed ids on the host
        raise ValueError("ids_host must be a contiguous int32 CPU tensor")
    out = torch.empty_like(x)
    arr, n = SlotCache._ids(prefetch or [])
    st = ex.struct()
    _lib.check(lib.moe_offload_layer_v1(
        pool.cache.handle, layer, x.data_ptr(), T, router_w.data_ptr(), ops._ptr(logit_bias),
        top_k, ctypes.byref(st), workspace.data_ptr(), ops._nbytes(workspace), out.data_ptr(),
        ids_host.data_ptr(), arr, n, p, ops._stream(), None))
    return out, ids_host


class OffloadDecoder:
    """Decode steps through offloaded MoE layers, with prefetch of predicted experts.

    Per layer, one moe_offload_layer_v1 call: router -> routed ids to the host -> demand (misses
    copied on the compute stream) -> experts from the layer's slots -> prefetch of the experts
    predicted for the next step on the copy streams (the demand's slots stay pinned, so no slot
    the layer's kernels read is overwritten) -> layer_done.
    Each layer reads the step's hidden state x (independent synthetic layers).
    """

    def __init__(self, pool: OffloadedExperts, routers: list[torch.Tensor],
                 biases: list[torch.Tensor | None], *, top_k: int = 8,
                 predictor: tuple[torch.Tensor, torch.Tensor] | None = None,
                 prefetch_k: int = 16, path: str = "auto") -> None:
        if len(routers) != pool.num_layers or len(biases) != pool.num_layers:
            raise ValueError("one router weight and bias per layer")
        self.pool, self.routers, self.biases = pool, routers, biases
        self.top_k, self.path, self.prefetch_k = top_k, path, prefetch_k
        self.predictor = predictor
        if isinstance(predictor, tuple):
            w1, w2 = predictor
            if w1.shape[0] != pool.num_layers or w2.shape[0] != pool.num_layers:
                raise ValueError("predictor needs one head per layer")
        elif predictor is not None and predictor.num_layers < pool.num_layers:
            raise ValueError("the predictor's layer embedding covers fewer layers than the pool")
        self._ids_host: torch.Tensor | None = None
        self._pred_host: torch.Tensor | None = None
        self._ws: torch.Tensor | None = None
        self._pred_ws: torch.Tensor | None = None
        self._lib = _lib.load()
        self._prepared: tuple | None = None
        self._layer_args: list[tuple] = []

    def predict(self, h: torch.Tensor) -> list[list[int]]:
        """Per layer, the distinct experts of the predictor's top-prefetch_k over h's rows.

        The predictor is either per-layer MLP heads (w1 [L, D, H], w2 [L, E, D]) or a
        HiddenResidualExpertPredictor, whose next-token delta (0) row for layer l is used."""
        if self.predictor is None or self.prefetch_k <= 0:
            return [[] for _ in range(self.pool.num_layers)]
        if not isinstance(self.predictor, tuple):
            L, T = self.pool.num_layers, h.shape[0]
            hh = h.repeat(L, 1)  # example (l, t) = row l * T + t
            lid = torch.arange(L, dtype=torch.int32, device=h.device).repeat_interleave(T)
            ids = self.predictor.predict_topk(hh, layer_ids=lid, k=self.prefetch_k)[:, 0, :]
            if self._pred_host is None or self._pred_host.shape != ids.shape:
                self._pred_host = torch.empty(ids.shape, dtype=torch.int32, pin_memory=True)
            self._pred_host.copy_(ids, non_blocking=True)
            torch.cuda.current_stream().synchronize()
            per = self._pred_host.view(L, T * self.prefetch_k)
            return [list(dict.fromkeys(per[l].tolist())) for l in range(L)]
        w1, w2 = self.predictor
        L, T, k = self.pool.num_layers, h.shape[0], self.prefetch_k
        need = ops.predictor_workspace_bytes(T, L, w1.shape[1], w2.shape[1], k)
        if self._pred_ws is None or self._pred_ws.numel() < need:
            self._pred_ws = torch.empty(need, dtype=torch.uint8, device=h.device)
        ids = ops.predictor_topk(h, w1, w2, k, workspace=self._pred_ws)
        if self._pred_host is None or self._pred_host.shape != ids.shape:
            self._pred_host = torch.empty(ids.shape, dtype=torch.int32, pin_memory=True)
        self._pred_host.copy_(ids, non_blocking=True)
        torch.cuda.current_stream().synchronize()
        return [list(dict.fromkeys(self._pred_host[l].reshape(-1).tolist())) for l in range(L)]

    def _prepare(self, x: torch.Tensor) -> None:
        """Checks of every layer's router and bias, the workspace, the pinned ids buffer and the
        per-layer call arguments, once per (batch size, device, top_k, path, router and bias
        tensors): a step's layer calls then run no Python checks (routed_layer's, done here for
        all layers at once). A router or bias replaced between steps is checked again."""
        key = (x.shape[0], x.device, self.top_k, self.path,
               tuple(r.data_ptr() for r in self.routers), tuple(map(ops._ptr, self.biases)))
        if self._prepared == key:
            return
        T, pool = x.shape[0], self.pool
        ex0 = pool.layer_experts(0)
        for l in range(pool.num_layers):
            ops._bf16_matrix(self.routers[l], "router_w", ex0.hidden_size)
            if self.routers[l].shape[0] != ex0.num_experts:
                raise ValueError(f"router_w of layer {l} has {self.routers[l].shape[0]} rows for "
                                 f"{ex0.num_experts} experts")
            ops._check_bias_gate(self.biases[l], None, ex0.num_experts, ex0.hidden_size)
            ops._require_gpu(x, self.routers[l], self.biases[l])
        p = ops._path(self.path)
        need = ops.workspace_bytes(T, self.top_k, ex0, False, p)
        if self._ws is None or self._ws.numel() < need or self._ws.device != x.device:
            self._ws = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
        self._ids_host = torch.empty((T, self.top_k), dtype=torch.int32, pin_memory=True)
        structs = [pool.layer_experts(l).struct() for l in range(pool.num_layers)]
        self._layer_args = [(self.routers[l].data_ptr(), ops._ptr(self.biases[l]), ctypes.byref(st),
                             st) for l, st in enumerate(structs)]
        self._path_id = p
        self._prepared = key

    def step(self, x: torch.Tensor, prefetch: list[list[int]] | None = None,
             trace: list | None = None) -> list[torch.Tensor]:
        """One decode step over every layer; `prefetch[l]` is issued right after layer l.
        Returns the layers' outputs (bf16 [T, H] each, views of one [L, T, H] tensor).

        trace: if given, one (layer, demanded experts, prefetched experts, host time in us)
        record per layer call is appended (the call's demand and prefetch happen inside it, after
        the routed ids reached the host), so the sequence can be replayed through the
        reference's virtual-time managers (mtp_amd.cache_manager)."""
        L, H = self.pool.num_layers, self.pool.hidden
        ops._bf16_matrix(x, "input", H)
        ops._require_gpu(x)
        if prefetch is not None and len(prefetch) < L:
            raise ValueError(f"prefetch lists for {len(prefetch)} of {L} layers")
        self._prepare(x)
        T = x.shape[0]
        out = torch.empty((L, T, H), dtype=torch.bfloat16, device=x.device)
        fn, check = self._lib.moe_offload_layer_v1, _lib.check
        handle, stream = self.pool.cache.handle, ops._stream()
        xp, op, row = x.data_ptr(), out.data_ptr(), T * H * 2
        wsp, wsn, ids = self._ws.data_ptr(), self._ws.numel(), self._ids_host.data_ptr()
        top_k, path = self.top_k, self._path_id
        for l, (rp, bp, sp, _) in enumerate(self._layer_args):
            pre = prefetch[l] if prefetch is not None else ()
            n = len(pre)
            arr = (ctypes.c_int32 * max(n, 1))(*map(int, pre))
            check(fn(handle, l, xp, T, rp, bp, top_k, sp, wsp, wsn, op + l * row, ids, arr, n,
                     path, stream, None))
            if trace is not None:
                trace.append((l, self._ids_host.reshape(-1).tolist(), list(pre),
                              time.perf_counter() * 1e6))
        return list(out.unbind(0))
