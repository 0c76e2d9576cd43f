"""Tensor-level wrappers of the C ABI. Every op runs the HIP kernels; none has a CPU path.

All tensors must live on one ROCm device; outputs are allocated with torch (caching
allocator, so the ops are safe to capture in a HIP graph) and every launch goes to
torch.cuda.current_stream().
"""

from __future__ import annotations

import ctypes

import torch

from mtp_amd import _lib
from mtp_amd.weights import MoeExperts

PATHS = {"auto": _lib.PATH_AUTO, "decode": _lib.PATH_DECODE, "prefill": _lib.PATH_PREFILL}
DECODE_BLOCK_M = 16
PREFILL_BLOCK_M = 128
AUTO_PREFILL_SLOTS = 2560  # routed slots (T * top_k) from which "auto" runs the prefill path
OUT_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_gpu(*tensors: torch.Tensor | None) -> None:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("the W4A16 MoE kernels need ROCm device tensors; got a CPU tensor")
        if not t.is_contiguous():
            raise ValueError("tensors passed to the W4A16 MoE kernels must be contiguous")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")


def _require_experts_on(device: torch.device, *sets: MoeExperts | None) -> None:
    """Expert sets are validated by MoeExperts.validate (contiguous stacks or slot-pool views);
    here only their device is checked against the activations'."""
    for ex in sets:
        if ex is not None and ex.device != device:
            raise ValueError(f"expert weights on {ex.device}, activations on {device}")


def _workspace(workspace: torch.Tensor | None, need: int, device: torch.device) -> torch.Tensor:
    """The caller's workspace when it is a contiguous tensor on ``device`` of at least ``need``
    bytes; a smaller one is replaced by a new allocation."""
    if workspace is not None:
        if not workspace.is_cuda or workspace.device != device or not workspace.is_contiguous():
            raise ValueError(f"workspace must be a contiguous tensor on {device}")
        if _nbytes(workspace) >= need:
            return workspace
    return torch.empty(max(need, 1), dtype=torch.uint8, device=device)


def _nbytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


def _path(path: str | int) -> int:
    if isinstance(path, int):
        return path
    try:
        return PATHS[path]
    except KeyError as exc:
        raise ValueError(f"path must be one of {sorted(PATHS)}") from exc


def _bf16_matrix(x: torch.Tensor, name: str, cols: int | None = None) -> None:
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {x.dtype}")
    if x.ndim != 2:
        raise ValueError(f"{name} must be 2D, got {tuple(x.shape)}")
    if cols is not None and x.shape[1] != cols:
        raise ValueError(f"Expected {name} last dim {cols}, got {x.shape[1]}")


def _check_bias_gate(logit_bias: torch.Tensor | None, shared_gate_w: torch.Tensor | None,
                     E: int, H: int) -> None:
    """The kernels read E float32 biases and H bf16 shared-gate weights."""
    if logit_bias is not None and (logit_bias.dtype != torch.float32 or logit_bias.numel() != E):
        raise ValueError("logit_bias must be float32 [E]")
    if shared_gate_w is not None and (shared_gate_w.dtype != torch.bfloat16
                                      or shared_gate_w.numel() != H):
        raise ValueError("shared_gate_w must be bfloat16 with hidden elements")


def _check_blocks(sorted_ids: torch.Tensor, expert_ids: torch.Tensor, ntpp: torch.Tensor,
                  block_m: int) -> None:
    """align's outputs as the grouped GEMMs read them: expert_ids.numel() blocks of block_m
    sorted slot ids and the padded total."""
    for name, t in (("sorted_ids", sorted_ids), ("expert_ids", expert_ids), ("ntpp", ntpp)):
        if t.dtype != torch.int32:
            raise TypeError(f"{name} must be int32")
    if sorted_ids.numel() < expert_ids.numel() * block_m or ntpp.numel() < 1:
        raise ValueError(f"sorted_ids holds {sorted_ids.numel()} ids for {expert_ids.numel()} "
                         f"blocks of {block_m}")


# ----------------------------------------------------------------------------- dequant
def dequantize(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
               g_idx: torch.Tensor | None = None, *, group_size: int = 128,
               linear_weight: bool = True, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """HIP dequant of one ([K/8, N]) or stacked ([E, K/8, N]) GPTQ projection.

    Bit-exact with dequantize_gptq_projection
    (src/mtp_expert_prefetch/repack/gptq_unpack.py:88-131)."""
    lib = _lib.load()
    squeeze = qweight.ndim == 2
    if squeeze:
        qweight, qzeros, scales = qweight[None], qzeros[None], scales[None]
        if g_idx is not None:
            g_idx = g_idx[None]
    _require_gpu(qweight, qzeros, scales, g_idx)
    if dtype not in OUT_DTYPES:
        raise ValueError(f"Unsupported dtype {dtype}")
    if qweight.ndim != 3 or qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
        raise TypeError("qweight [E, K/8, N] and qzeros must be int32")
    if scales.dtype != torch.float16:
        raise TypeError(f"scales must be float16, got {scales.dtype}")
    e, k8, n = qweight.shape
    k = k8 * 8
    if group_size <= 0 or k % group_size != 0:
        raise ValueError(f"group_size {group_size} does not divide in_features {k}")
    ng = k // group_size
    if tuple(scales.shape) != (e, ng, n) or tuple(qzeros.shape) != (e, ng, n // 8):
        raise ValueError(f"scales {tuple(scales.shape)} / qzeros {tuple(qzeros.shape)} do not "
                         f"match qweight {tuple(qweight.shape)} with group_size {group_size}")
    if g_idx is not None:
        if tuple(g_idx.shape) != (e, k):
            raise ValueError(f"g_idx {tuple(g_idx.shape)} must be [E, K] = {(e, k)}")
        lo, hi = (int(v) for v in torch.aminmax(g_idx))
        if lo < 0 or hi >= ng:  # the kernel reads the scales and zeros row g_idx[k]
            raise ValueError(f"g_idx out of range [{lo}, {hi}] for {ng} groups")
    out_shape = (e, n, k) if linear_weight else (e, k, n)
    out = torch.empty(out_shape, dtype=dtype, device=qweight.device)
    proj = _lib.GptqProj(qweight.data_ptr(), qzeros.data_ptr(), scales.data_ptr())
    gi = None
    if g_idx is not None:
        gi = g_idx.to(torch.int32).contiguous()
    _lib.check(lib.moe_dequant_v1(ctypes.byref(proj), _ptr(gi), e, k, n, group_size,
                                  1 if linear_weight else 0, OUT_DTYPES[dtype], out.data_ptr(),
                                  _stream()))
    return out[0] if squeeze else out


# ----------------------------------------------------------------------------- router
def router_topk(x: torch.Tensor, router_w: torch.Tensor, top_k: int = 8, *,
                logit_bias: torch.Tensor | None = None,
                shared_gate_w: torch.Tensor | None = None):
    """fp32 logits -> softmax -> top-k -> renormalise (bit-exact ids, ties to the lower id).

    Returns (topk_ids int32 [T, k], topk_weights fp32 [T, k], shared_gate fp32 [T] or None,
    logits fp32 [T, E])."""
    lib = _lib.load()
    _bf16_matrix(x, "input")
    _bf16_matrix(router_w, "router_w", x.shape[1])
    _require_gpu(x, router_w, logit_bias, shared_gate_w)
    T, E = x.shape[0], router_w.shape[0]
    if not 0 < top_k <= E:
        raise ValueError(f"top_k must be in [1, {E}], got {top_k}")
    dev = x.device
    logits = torch.empty(T, E + 1, dtype=torch.float32, device=dev)
    ids = torch.empty(T, top_k, dtype=torch.int32, device=dev)
    has_shared = shared_gate_w is not None
    w = torch.empty(T * top_k + (T if has_shared else 0), dtype=torch.float32, device=dev)
    if logit_bias is not None and (logit_bias.dtype != torch.float32 or logit_bias.numel() != E):
        raise ValueError("logit_bias must be float32 [E]")
    if has_shared:
        if shared_gate_w.dtype != torch.bfloat16 or shared_gate_w.numel() != x.shape[1]:
            raise ValueError("shared_gate_w must be bfloat16 with hidden elements")
    _lib.check(lib.moe_router_topk_v1(x.data_ptr(), T, x.shape[1], router_w.data_ptr(), E,
                                      _ptr(logit_bias), top_k, _ptr(shared_gate_w),
                                      logits.data_ptr(), ids.data_ptr(), w.data_ptr(), _stream()))
    topk_w = w[: T * top_k].view(T, top_k)
    shared = w[T * top_k:] if has_shared else None
    return ids, topk_w, shared, logits[:, :E]


# ----------------------------------------------------------------------------- align
def capacity_blocks(T: int, top_k: int, num_experts: int, has_shared: bool, block_m: int) -> int:
    return int(_lib.load().moe_capacity_blocks_v1(T, top_k, num_experts, int(has_shared), block_m))


def align(topk_ids: torch.Tensor, num_experts: int, block_m: int, *, has_shared: bool = False,
          capacity: int | None = None):
    """Block-padded expert-grouped slot permutation (vLLM moe_align_block_size format)."""
    lib = _lib.load()
    if topk_ids.dtype != torch.int32 or topk_ids.ndim != 2:
        raise TypeError("topk_ids must be int32 [T, k]")
    _require_gpu(topk_ids)
    T, k = topk_ids.shape
    cap = capacity if capacity is not None else capacity_blocks(T, k, num_experts, has_shared, block_m)
    dev = topk_ids.device
    sorted_ids = torch.empty(cap * block_m, dtype=torch.int32, device=dev)
    eids = torch.empty(cap, dtype=torch.int32, device=dev)
    ntpp = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.check(lib.moe_align_v1(topk_ids.data_ptr(), T, k, num_experts, int(has_shared), block_m,
                                cap, sorted_ids.data_ptr(), eids.data_ptr(), ntpp.data_ptr(),
                                _stream()))
    return sorted_ids, eids, ntpp


# ----------------------------------------------------------------------------- GEMMs
def _block_m(path: int, T: int, top_k: int) -> int:
    if path == _lib.PATH_AUTO:
        path = _lib.PATH_PREFILL if T * top_k >= AUTO_PREFILL_SLOTS else _lib.PATH_DECODE
    return PREFILL_BLOCK_M if path == _lib.PATH_PREFILL else DECODE_BLOCK_M


def w1_gateup_silu(x, experts: MoeExperts, sorted_ids, expert_ids, ntpp, *, top_k: int,
                   shared: MoeExperts | None = None, path: str | int = "auto") -> torch.Tensor:
    lib = _lib.load()
    p = _path(path)
    _bf16_matrix(x, "input", experts.hidden_size)
    _require_gpu(x, sorted_ids, expert_ids, ntpp)
    _require_experts_on(x.device, experts, shared)
    T = x.shape[0]
    bm = _block_m(p, T, top_k)
    _check_blocks(sorted_ids, expert_ids, ntpp, bm)
    slots = T * top_k + (T if shared is not None else 0)
    h = torch.empty(slots, experts.intermediate_size, dtype=torch.bfloat16, device=x.device)
    ex = experts.struct()
    sh = shared.struct() if shared is not None else None
    _lib.check(lib.moe_w1_gateup_silu_v1(
        x.data_ptr(), T, top_k, ctypes.byref(ex), ctypes.byref(sh) if sh else None,
        sorted_ids.data_ptr(), expert_ids.data_ptr(), ntpp.data_ptr(), bm, expert_ids.numel(),
        h.data_ptr(), p, _stream()))
    return h


def w2_down(h, experts: MoeExperts, sorted_ids, expert_ids, ntpp, topk_weights_flat, *, T: int,
            top_k: int, shared: MoeExperts | None = None, path: str | int = "auto",
            ys: torch.Tensor | None = None) -> torch.Tensor:
    """Weighted W2 rows ys fp32 [slots, H]; rows of dropped slots are left as they were."""
    lib = _lib.load()
    p = _path(path)
    slots = T * top_k + (T if shared is not None else 0)
    _bf16_matrix(h, "h", experts.intermediate_size)
    if h.shape[0] < slots:
        raise ValueError(f"h has {h.shape[0]} rows for {slots} slots")
    if topk_weights_flat.dtype != torch.float32 or topk_weights_flat.numel() < slots:
        raise ValueError(f"topk_weights_flat must be float32 with at least {slots} elements")
    _require_gpu(h, sorted_ids, expert_ids, ntpp, topk_weights_flat)
    _require_experts_on(h.device, experts, shared)
    bm = _block_m(p, T, top_k)
    _check_blocks(sorted_ids, expert_ids, ntpp, bm)
    if ys is None:
        ys = torch.empty(h.shape[0], experts.hidden_size, dtype=torch.float32, device=h.device)
    elif (ys.dtype != torch.float32 or tuple(ys.shape) != (h.shape[0], experts.hidden_size)
          or not ys.is_contiguous()):
        raise ValueError("ys must be contiguous float32 [slots, hidden]")
    _require_gpu(h, ys)
    ex = experts.struct()
    sh = shared.struct() if shared is not None else None
    _lib.check(lib.moe_w2_down_v1(
        h.data_ptr(), T, top_k, ctypes.byref(ex), ctypes.byref(sh) if sh else None,
        sorted_ids.data_ptr(), expert_ids.data_ptr(), ntpp.data_ptr(), bm, expert_ids.numel(),
        topk_weights_flat.data_ptr(), ys.data_ptr(), p, _stream()))
    return ys


def moe_sum(ys: torch.Tensor, topk_ids: torch.Tensor, experts: MoeExperts,
            has_shared: bool = False) -> torch.Tensor:
    """Fixed-order fp32 sum of each token's weighted W2 rows -> bf16 [T, H]. Slots whose id is
    outside [0, E) or whose expert is not resident in a slot pool are skipped (w2_down leaves
    their rows unwritten)."""
    lib = _lib.load()
    if topk_ids.dtype != torch.int32 or topk_ids.ndim != 2:
        raise TypeError("topk_ids must be int32 [T, k]")
    _require_gpu(ys, topk_ids)
    T, top_k = topk_ids.shape
    H = ys.shape[1]
    if (ys.dtype != torch.float32 or ys.ndim != 2
            or ys.shape[0] < T * top_k + (T if has_shared else 0)):
        raise ValueError("ys must be float32 [T*k (+T), H]")
    out = torch.empty(T, H, dtype=torch.bfloat16, device=ys.device)
    _lib.check(lib.moe_sum_v1(ys.data_ptr(), T, top_k, H, int(has_shared), topk_ids.data_ptr(),
                              int(experts.num_experts), _ptr(experts.expert_row), out.data_ptr(),
                              _stream()))
    return out


# ----------------------------------------------------------------------------- decoder norm
def rmsnorm(res: torch.Tensor, weight: torch.Tensor, *, add: torch.Tensor | None = None,
            eps: float = 1e-6, out: torch.Tensor | None = None) -> torch.Tensor:
    """Residual add (in place into ``res`` when ``add`` is given) and the (1 + w) RMSNorm of
    mtp_rms_norm (src/mtp_expert_prefetch/mtp/extra_tensors.py:40-48) on the HIP kernel.

    res, add: bf16 [T, hidden]; weight bf16 [hidden]. Returns bf16 [T, hidden]."""
    lib = _lib.load()
    _bf16_matrix(res, "res")
    T, H = res.shape
    if add is not None:
        _bf16_matrix(add, "add", H)
        if add.shape[0] != T:
            raise ValueError(f"add has {add.shape[0]} rows for {T}")
    if weight.dtype != torch.bfloat16 or weight.numel() != H or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous bfloat16 tensor of hidden elements")
    _require_gpu(res, add, weight)
    if out is None:
        out = torch.empty_like(res)
    elif out.shape != res.shape or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous bf16 tensor shaped like res")
    _require_gpu(res, out)
    _lib.check(lib.moe_rmsnorm_v1(res.data_ptr(), _ptr(add), T, H, weight.data_ptr(), float(eps),
                                  out.data_ptr(), _stream()))
    return out


# ----------------------------------------------------------------------------- whole layer
def workspace_bytes(T: int, top_k: int, experts: MoeExperts, has_shared: bool,
                    path: str | int = "auto") -> int:
    ex = experts.struct()
    n = int(_lib.load().moe_layer_workspace_bytes_v1(T, top_k, ctypes.byref(ex), int(has_shared),
                                                     _path(path)))
    if n < 0:
        raise ValueError("invalid sizes for the workspace query")
    return n


def moe_layer(x: torch.Tensor, router_w: torch.Tensor, experts: MoeExperts, *, top_k: int = 8,
              logit_bias: torch.Tensor | None = None, shared: MoeExperts | None = None,
              shared_gate_w: torch.Tensor | None = None, path: str | int = "auto",
              workspace: torch.Tensor | None = None, return_routing: bool = False,
              out: torch.Tensor | None = None):
    """Routed MoE layer: router -> align -> W1 -> W2 -> sum (+ gated shared expert)."""
    lib = _lib.load()
    _bf16_matrix(x, "input", experts.hidden_size)
    _bf16_matrix(router_w, "router_w", experts.hidden_size)
    if router_w.shape[0] != experts.num_experts:
        raise ValueError(f"router_w has {router_w.shape[0]} rows for {experts.num_experts} experts")
    if (shared is None) != (shared_gate_w is None):
        raise ValueError("shared and shared_gate_w must be given together")
    _check_bias_gate(logit_bias, shared_gate_w, experts.num_experts, experts.hidden_size)
    _require_gpu(x, router_w, logit_bias, shared_gate_w)
    _require_experts_on(x.device, experts, shared)
    T = x.shape[0]
    p = _path(path)
    workspace = _workspace(workspace, workspace_bytes(T, top_k, experts, shared is not None, p),
                           x.device)
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous bf16 tensor shaped like the input")
    _require_gpu(x, out)
    ids = torch.empty(T, top_k, dtype=torch.int32, device=x.device) if return_routing else None
    w = torch.empty(T, top_k, dtype=torch.float32, device=x.device) if return_routing else None
    ex = experts.struct()
    sh = shared.struct() if shared is not None else None
    _lib.check(lib.moe_layer_v1(
        x.data_ptr(), T, router_w.data_ptr(), _ptr(logit_bias), top_k, ctypes.byref(ex),
        ctypes.byref(sh) if sh else None, _ptr(shared_gate_w), workspace.data_ptr(),
        _nbytes(workspace), out.data_ptr(), _ptr(ids), _ptr(w), p, _stream()))
    if return_routing:
        return out, ids, w
    return out


def norm_layer(res: torch.Tensor, router_w: torch.Tensor, experts: MoeExperts,
               norm_w: torch.Tensor, *, add: torch.Tensor | None = None, eps: float = 1e-6,
               res_out: torch.Tensor | None = None, x_out: torch.Tensor | None = None,
               top_k: int = 8, logit_bias: torch.Tensor | None = None,
               shared: MoeExperts | None = None, shared_gate_w: torch.Tensor | None = None,
               path: str | int = "auto", workspace: torch.Tensor | None = None,
               out: torch.Tensor | None = None):
    """A decoder step: res_out = res + add, x = rmsnorm(res_out) * (1 + norm_w), then the routed
    layer on x (moe_norm_layer_v1; the bits of ``rmsnorm`` followed by ``moe_layer``). Returns
    (out, res_out, x). res_out defaults to a new tensor (a distinct buffer lets decode batches
    normalise inside the router); pass ``res`` itself to update it in place."""
    lib = _lib.load()
    _bf16_matrix(res, "res", experts.hidden_size)
    _bf16_matrix(router_w, "router_w", experts.hidden_size)
    T, H = res.shape
    if add is not None:
        _bf16_matrix(add, "add", H)
        if add.shape[0] != T:
            raise ValueError(f"add has {add.shape[0]} rows for {T}")
    if norm_w.dtype != torch.bfloat16 or norm_w.numel() != H or not norm_w.is_contiguous():
        raise ValueError("norm_w must be a contiguous bfloat16 tensor of hidden elements")
    if (shared is None) != (shared_gate_w is None):
        raise ValueError("shared and shared_gate_w must be given together")
    _check_bias_gate(logit_bias, shared_gate_w, experts.num_experts, experts.hidden_size)
    _require_gpu(res, add, norm_w, router_w, logit_bias, shared_gate_w)
    _require_experts_on(res.device, experts, shared)
    if res_out is None:
        res_out = torch.empty_like(res)
    if x_out is None:
        x_out = torch.empty_like(res)
    if out is None:
        out = torch.empty_like(res)
    for t, name in ((res_out, "res_out"), (x_out, "x_out"), (out, "out")):
        if t.shape != res.shape or t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous bf16 tensor shaped like res")
    _require_gpu(res, res_out, x_out, out)
    p = _path(path)
    workspace = _workspace(workspace, workspace_bytes(T, top_k, experts, shared is not None, p),
                           res.device)
    ex = experts.struct()
    sh = shared.struct() if shared is not None else None
    _lib.check(lib.moe_norm_layer_v1(
        res.data_ptr(), _ptr(add), norm_w.data_ptr(), float(eps), res_out.data_ptr(),
        x_out.data_ptr(), T, router_w.data_ptr(), _ptr(logit_bias), top_k, ctypes.byref(ex),
        ctypes.byref(sh) if sh else None, _ptr(shared_gate_w), workspace.data_ptr(),
        _nbytes(workspace), out.data_ptr(), None, None, p, _stream()))
    return out, res_out, x_out


def fused_experts(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                  experts: MoeExperts, *, shared: MoeExperts | None = None,
                  shared_gate_w: torch.Tensor | None = None, path: str | int = "auto",
                  workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Experts with caller-given routing (ids int32 [T, k], weights fp32 [T, k])."""
    lib = _lib.load()
    _bf16_matrix(x, "input", experts.hidden_size)
    if topk_ids.dtype != torch.int32 or topk_weights.dtype != torch.float32:
        raise TypeError("topk_ids must be int32 and topk_weights float32")
    if topk_ids.shape != topk_weights.shape or topk_ids.ndim != 2 or topk_ids.shape[0] != x.shape[0]:
        raise ValueError("topk_ids/topk_weights must be [T, k] matching the input rows")
    if (shared is None) != (shared_gate_w is None):
        raise ValueError("shared and shared_gate_w must be given together")
    _check_bias_gate(None, shared_gate_w, experts.num_experts, experts.hidden_size)
    _require_gpu(x, topk_ids, topk_weights, shared_gate_w)
    _require_experts_on(x.device, experts, shared)
    T, k = topk_ids.shape
    p = _path(path)
    workspace = _workspace(workspace, workspace_bytes(T, k, experts, shared is not None, p),
                           x.device)
    out = torch.empty_like(x)
    ex = experts.struct()
    sh = shared.struct() if shared is not None else None
    _lib.check(lib.moe_fused_experts_v1(
        x.data_ptr(), T, topk_ids.data_ptr(), topk_weights.data_ptr(), k, ctypes.byref(ex),
        ctypes.byref(sh) if sh else None, _ptr(shared_gate_w), workspace.data_ptr(),
        _nbytes(workspace), out.data_ptr(), p, _stream()))
    return out


# ----------------------------------------------------------------------------- predictor
def predictor_workspace_bytes(T: int, num_heads: int, inner: int, num_experts: int, top_k: int) -> int:
    return int(_lib.load().moe_predictor_workspace_bytes_v1(T, num_heads, inner, num_experts, top_k))


def predictor_topk(h: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, top_k: int = 16, *,
                   workspace: torch.Tensor | None = None,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-layer predicted experts: int32 [L, T, top_k] from h bf16 [T, H], w1 bf16 [L, D, H]
    (or [D, H] for one head), w2 bf16 [L, E, D] (or [E, D]).

    Each head computes bf16(silu(h . w1[l]^T)) . w2[l]^T in fp32 and keeps its top-k by
    (logit desc, id asc); the reference's per-layer predictor head
    (src/mtp_expert_prefetch/training/hidden_residual.py:44-106) simplified to hidden -> inner
    (SiLU) -> experts.
    """
    lib = _lib.load()
    if w1.dim() == 2:
        w1 = w1.unsqueeze(0)
    if w2.dim() == 2:
        w2 = w2.unsqueeze(0)
    _bf16_matrix(h, "hidden")
    if w1.dim() != 3 or w2.dim() != 3 or w1.shape[0] != w2.shape[0]:
        raise ValueError("w1 must be [L, D, H] and w2 [L, E, D] with the same L")
    L, D, H = w1.shape
    E = w2.shape[1]
    if H != h.shape[1] or w2.shape[2] != D:
        raise ValueError(f"predictor shapes: h {tuple(h.shape)}, w1 {tuple(w1.shape)}, w2 {tuple(w2.shape)}")
    for t, name in ((w1, "w1"), (w2, "w2")):
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise TypeError(f"{name} must be contiguous bf16")
    _require_gpu(h, w1, w2)
    T = h.shape[0]
    # a negative size (invalid sizes) leaves the error to the entry point's own checks
    workspace = _workspace(workspace, predictor_workspace_bytes(T, L, D, E, top_k), h.device)
    if out is None:
        out = torch.empty(L, T, top_k, dtype=torch.int32, device=h.device)
    elif out.dtype != torch.int32 or out.shape != (L, T, top_k) or not out.is_contiguous():
        raise ValueError("out must be contiguous int32 [L, T, top_k]")
    _require_gpu(h, out)
    _lib.check(lib.moe_predictor_v1(h.data_ptr(), T, H, L, w1.data_ptr(), D, w2.data_ptr(), E,
                                    top_k, workspace.data_ptr(), _nbytes(workspace),
                                    out.data_ptr(), _stream()))
    return out
