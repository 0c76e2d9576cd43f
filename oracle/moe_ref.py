"""Router, align/sort, expert MLP and the full MoE layer, restated on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference semantics followed (paths relative to the reference repo root):
  router       tracing/vllm_router_trace.py:4201-4225 (topk_softmax, renormalize=True):
               p = softmax_fp32(logits); top-k; w = p_top / max(sum p_top, 1e-20).
               Because renormalisation cancels the full softmax denominator this is
               w_i = exp(l_i - l_max) / sum_{j in top-k} exp(l_j - l_max).
               Tie rule (explicit, replaces torch.topk's unspecified order): larger
               logit first, equal logits -> lower expert id first.
  logits       x . W_r^T with fp32 accumulation in one canonical order (below) so that
               the HIP router kernel and this oracle produce identical fp32 logits.
  align        vLLM moe_align_block_size format as used at vllm_router_trace.py:19647-19660
               and restated at tracing/vllm_wna16_group_plan.py:68-132: flat slot ids
               grouped by expert, each group padded to block_m with the sentinel
               ``num_slots``, one expert id per block, num_tokens_post_padded.
               Order inside the format is defined stably: experts ascending, slots
               ascending (a stable argsort).
  expert MLP   repack/gptq_unpack.py:247-256  y = W_down (silu(W_gate x) * (W_up x))
  top-k sum    repack/gptq_unpack.py:293-327 and mtp/extra_tensors.py:544-598
               out[t] = sum_i w[t,i] * expert_{id[t,i]}(x[t])  (+ shared expert:
               sigmoid(x . w_g) * shared(x), extra_tensors.py:596-597)
  silu_and_mul vllm_router_trace.py:4178-4180 (gate = first half)

Canonical logit order (shared with the router kernel): K is cut into chunks of 8
consecutive elements; chunk q belongs to lane q % 64. Each lane accumulates its
chunks in increasing q, elements in increasing k, starting from +0.0f, with
acc = fma(x, w, acc); bf16 x bf16 products are exact in fp32, so this equals
acc + x*w evaluated in float32. The 64 lane partials are combined by the butterfly
v += shfl_xor(v, m) for m = 32, 16, 8, 4, 2, 1.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import gptq_ref

LANES = 64


# --------------------------------------------------------------------------- router
def canonical_dot_rows(x_f32: np.ndarray, w_f32: np.ndarray) -> np.ndarray:
    """Canonical-order fp32 dot products: out[t, e] = sum_k x[t, k] * w[e, k].

    x_f32 [T, K] and w_f32 [E, K] hold bf16-representable values; K % 8 == 0.
    """
    T, K = x_f32.shape
    E = w_f32.shape[0]
    assert K % 8 == 0
    nq = K // 8
    nc = -(-nq // LANES)
    # pad K to nc*64*8 with zeros; a zero product adds +0.0 and leaves acc unchanged
    pad = nc * LANES * 8 - K
    xp = np.pad(x_f32.astype(np.float32), ((0, 0), (0, pad)))
    wp = np.pad(w_f32.astype(np.float32), ((0, 0), (0, pad)))
    # [T, nc, 64, 8] chunk layout: k = (c*64 + lane)*8 + i
    xr = xp.reshape(T, nc, LANES, 8)
    wr = wp.reshape(E, nc, LANES, 8)
    acc = np.zeros((T, E, LANES), dtype=np.float32)
    for c in range(nc):
        for i in range(8):
            prod = (xr[:, None, c, :, i] * wr[None, :, c, :, i]).astype(np.float32)
            acc = (acc + prod).astype(np.float32)
    v = acc
    width = LANES
    while width > 1:
        half = width // 2
        v = (v[..., :half] + v[..., half:width]).astype(np.float32)
        width = half
    return v[..., 0]


def router_logits(x_bits: np.ndarray, router_w_bits: np.ndarray,
                  logit_bias: np.ndarray | None = None) -> np.ndarray:
    """fp32 router logits [T, E] from bf16 bits (extra_tensors.py:353, fp32 accumulation)."""
    logits = canonical_dot_rows(gptq_ref.bf16_bits_to_f32(x_bits), gptq_ref.bf16_bits_to_f32(router_w_bits))
    if logit_bias is not None:
        logits = (logits + logit_bias.astype(np.float32)[None, :]).astype(np.float32)
    return logits


def stable_topk(logits: np.ndarray, k: int) -> np.ndarray:
    """Top-k ids per row: larger value first, ties -> lower id (lexsort on (id, -value))."""
    T, E = logits.shape
    ids = np.empty((T, k), dtype=np.int32)
    for t in range(T):
        order = np.lexsort((np.arange(E), -logits[t].astype(np.float64)))
        ids[t] = order[:k]
    return ids


def renorm_weights(logits: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """w_i = exp(l_i - l_top1) / sum_j exp(l_j - l_top1), fp32, j in rank order."""
    sel = np.take_along_axis(logits, ids.astype(np.int64), axis=1).astype(np.float32)
    e = np.exp((sel - sel[:, :1]).astype(np.float32)).astype(np.float32)
    s = np.zeros(sel.shape[0], dtype=np.float32)
    for i in range(sel.shape[1]):
        s = (s + e[:, i]).astype(np.float32)
    return (e / s[:, None]).astype(np.float32)


def router_topk(x_bits, router_w_bits, top_k=8, logit_bias=None):
    """Returns (ids [T,k] int32, weights [T,k] fp32, logits [T,E] fp32)."""
    logits = router_logits(x_bits, router_w_bits, logit_bias)
    ids = stable_topk(logits, top_k)
    return ids, renorm_weights(logits, ids), logits


def shared_gate(x_bits: np.ndarray, gate_w_bits: np.ndarray) -> np.ndarray:
    """sigmoid(x . w_g) in fp32 with the canonical dot order (extra_tensors.py:596)."""
    v = canonical_dot_rows(gptq_ref.bf16_bits_to_f32(x_bits), gptq_ref.bf16_bits_to_f32(gate_w_bits).reshape(1, -1))[:, 0]
    return (1.0 / (1.0 + np.exp(-v.astype(np.float64)))).astype(np.float32)


# --------------------------------------------------------------------------- align
def align_block_padded(topk_ids: np.ndarray, num_experts: int, block_m: int,
                       *, has_shared: bool = False, capacity_blocks: int | None = None):
    """Block-padded, expert-grouped permutation of flat slot ids.

    Slots: f = t*k + i for the routed choices; with ``has_shared`` every token t also
    owns slot T*k + t routed to expert id ``num_experts`` (the shared expert).
    Returns (sorted_token_ids [capacity*block_m], expert_ids [capacity], ntpp) with
    sentinel = number of slots; unused blocks carry expert id -1.
    """
    T, k = topk_ids.shape
    flat = topk_ids.reshape(-1).astype(np.int64)
    if has_shared:
        flat = np.concatenate([flat, np.full(T, num_experts, dtype=np.int64)])
    n_slots = flat.shape[0]
    n_exp = num_experts + (1 if has_shared else 0)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=n_exp)
    padded = -(-counts // block_m) * block_m
    ntpp = int(padded.sum())
    n_blocks = ntpp // block_m
    if capacity_blocks is None:
        capacity_blocks = n_blocks
    assert capacity_blocks >= n_blocks
    sorted_ids = np.full(capacity_blocks * block_m, n_slots, dtype=np.int32)
    expert_ids = np.full(capacity_blocks, -1, dtype=np.int32)
    pos = 0
    src = 0
    for e in range(n_exp):
        c = int(counts[e])
        if c == 0:
            continue
        sorted_ids[pos:pos + c] = order[src:src + c]
        expert_ids[pos // block_m:(pos + int(padded[e])) // block_m] = e
        pos += int(padded[e])
        src += c
    return sorted_ids, expert_ids, ntpp


def max_blocks(num_slots: int, num_groups: int, block_m: int) -> int:
    """Upper bound on sum_e ceil(n_e / block_m) over at most num_groups non-empty groups."""
    return -(-num_slots // block_m) + min(num_groups, num_slots)


# --------------------------------------------------------------------------- experts
def dequant_expert(layer: dict, e: int, prefix: str = "") -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """bf16-exact dequantised (gate, up, down) Linear weights of expert e as fp32 tensors."""
    out = []
    for proj in ("gate_proj", "up_proj", "down_proj"):
        bits = gptq_ref.dequant_bf16_bits(
            layer[f"{prefix}{proj}.qweight"][e], layer[f"{prefix}{proj}.qzeros"][e],
            layer[f"{prefix}{proj}.scales"][e], group_size=layer.get("group_size", 128))
        out.append(torch.from_numpy(gptq_ref.bf16_bits_to_f32(bits)))
    return tuple(out)


def expert_mlp_f32(x: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, wd: torch.Tensor) -> torch.Tensor:
    """SingleExpertMlp.forward in fp32 (gptq_unpack.py:247-256)."""
    g = x @ wg.T
    u = x @ wu.T
    return (F.silu(g) * u) @ wd.T


def moe_layer_f32(x_bits: np.ndarray, ids: np.ndarray, weights: np.ndarray, layer: dict,
                  *, shared: dict | None = None, shared_gate_values: np.ndarray | None = None,
                  dropped: frozenset[int] = frozenset()) -> np.ndarray:
    """fp32-accumulated top-k expert sum (+ gated shared expert), slot order i = 0..k-1.

    layer holds numpy arrays keyed '{proj}.{kind}' stacked over experts [E, ...]. A slot whose
    id is outside [0, E), or names an expert in `dropped`, contributes nothing (the reference
    drops ids outside [0, E) and unmapped experts, vllm_router_trace.py:14138-14153).
    """
    x = torch.from_numpy(gptq_ref.bf16_bits_to_f32(x_bits))
    T, H = x.shape
    E = layer["gate_proj.qweight"].shape[0]
    out = torch.zeros(T, H, dtype=torch.float32)
    keep = [int(e) for e in np.unique(ids) if 0 <= int(e) < E and int(e) not in dropped]
    cache: dict[int, tuple] = {e: dequant_expert(layer, e) for e in keep}
    for i in range(ids.shape[1]):
        for e in np.unique(ids[:, i]):
            if int(e) not in cache:
                continue
            rows = np.nonzero(ids[:, i] == e)[0]
            y = expert_mlp_f32(x[rows], *cache[int(e)])
            out[rows] += torch.from_numpy(weights[rows, i]).float()[:, None] * y
    if shared is not None:
        sg = torch.from_numpy(shared_gate_values).float()[:, None]
        out += sg * expert_mlp_f32(x, *dequant_expert(shared, 0))
    return out.numpy()


def moe_layer_ref(x_bits, router_w_bits, layer, *, top_k=8, logit_bias=None,
                  shared=None, shared_gate_w_bits=None):
    """Full layer oracle: (out_f32 [T,H], ids, weights, shared_gate_or_None)."""
    ids, w, _ = router_topk(x_bits, router_w_bits, top_k, logit_bias)
    sg = None
    if shared is not None:
        sg = shared_gate(x_bits, shared_gate_w_bits)
    out = moe_layer_f32(x_bits, ids, w, layer, shared=shared, shared_gate_values=sg)
    return out, ids, w, sg


def rel_err(out: np.ndarray, ref: np.ndarray) -> float:
    """Normwise max relative error max|out - ref| / max|ref| (the layer tolerance metric)."""
    denom = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(out.astype(np.float64) - ref.astype(np.float64)))) / max(denom, 1e-30)


# --------------------------------------------------------------------------- faithful bf16 path
def dequant_stack_torch(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                        group_size: int = 128) -> torch.Tensor:
    """Vectorised CPU dequant of stacked experts -> bf16 Linear weights [n, N, K].

    Same formula as gptq_ref.dequant_bf16_bits (gptq_unpack.py:88-131), in torch for speed;
    pinned bit-for-bit against the numpy restatement in tests/test_oracle_moe.py."""
    n, k8, cols = qweight.shape
    u = qweight.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(8, dtype=torch.int64) * 4
    q = ((u[:, :, None, :] >> shifts[None, None, :, None]) & 0xF).reshape(n, k8 * 8, cols)
    zu = qzeros.to(torch.int64) & 0xFFFFFFFF
    z = ((zu[:, :, :, None] >> shifts[None, None, None, :]) & 0xF).reshape(n, qzeros.shape[1], cols)
    g = torch.arange(k8 * 8) // group_size
    w = (q.to(torch.float32) - z.to(torch.float32)[:, g, :]) * scales.to(torch.float32)[:, g, :]
    return w.transpose(1, 2).contiguous().to(torch.bfloat16)



def moe_tokens_bf16(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
                    experts: dict[int, tuple[torch.Tensor, torch.Tensor, torch.Tensor]],
                    shared: tuple | None = None, shared_gate_w: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's own dtype flow on the CPU (extra_tensors.py:544-598):
    bf16 F.linear per expert, slot x unique-expert loop, output accumulated in bf16.
    Used as the timed CPU baseline, not as the parity reference."""
    flat_x = x.reshape(-1, x.shape[-1])
    output = torch.zeros_like(flat_x)
    for slot in range(ids.shape[1]):
        slot_ids = ids[:, slot]
        slot_w = weights[:, slot].to(flat_x.dtype)
        for e in torch.unique(slot_ids).tolist():
            mask = slot_ids == e
            wg, wu, wd = experts[int(e)]
            xm = flat_x[mask]
            y = F.linear(F.silu(F.linear(xm, wg)) * F.linear(xm, wu), wd)
            output[mask] = output[mask] + slot_w[mask, None] * y
    if shared is not None:
        wg, wu, wd = shared
        sg = torch.sigmoid(F.linear(flat_x, shared_gate_w))
        output = output + sg * F.linear(F.silu(F.linear(flat_x, wg)) * F.linear(flat_x, wu), wd)
    return output.reshape_as(x)


# --------------------------------------------------------------------------- predictor
def predictor_ref(h_bits: np.ndarray, w1_bits: np.ndarray, w2_bits: np.ndarray, top_k: int):
    """Per-layer predictor heads (training/hidden_residual.py:44-106, simplified to
    hidden -> inner SiLU -> experts): z1 = h . w1[l]^T (canonical fp32 order),
    a = bf16_RNE(z1 / (1 + exp(-z1))) in fp32, logits = a . w2[l]^T (canonical order),
    ids = stable top-k. h_bits [T, H]; w1_bits [L, D, H]; w2_bits [L, E, D].
    Returns (ids int32 [L, T, k], logits fp32 [L, T, E])."""
    h = gptq_ref.bf16_bits_to_f32(h_bits)
    L = w1_bits.shape[0]
    ids, logits = [], []
    for l in range(L):
        z1 = canonical_dot_rows(h, gptq_ref.bf16_bits_to_f32(w1_bits[l]))
        act = (z1 / (np.float32(1.0) + np.exp(-z1))).astype(np.float32)
        a = gptq_ref.bf16_bits_to_f32(gptq_ref.f32_to_bf16_bits(act))
        z2 = canonical_dot_rows(a, gptq_ref.bf16_bits_to_f32(w2_bits[l]))
        logits.append(z2)
        ids.append(stable_topk(z2, top_k))
    return np.stack(ids), np.stack(logits)


def rmsnorm_ref(res_bits: np.ndarray, weight_bits: np.ndarray, *, add_bits: np.ndarray | None = None,
                eps: float = 1e-6) -> tuple[np.ndarray, np.ndarray]:
    """Residual add and mtp_rms_norm (mtp/extra_tensors.py:40-48) in float32.

    res' = bf16(res + add) (fp32 add, round to nearest even) when add is given; then
    out = bf16((res' * rsqrt(mean(res'^2) + eps)) * (1 + w)), every step in float32 as the
    reference's fp32 variance and (1 + weight) scaling. Returns (res' bits, out bits); the mean
    is a float64 sum rounded to float32 (the HIP kernel sums in fp32 in its own fixed order)."""
    x = gptq_ref.bf16_bits_to_f32(res_bits)
    if add_bits is not None:
        x = gptq_ref.bf16_bits_to_f32(gptq_ref.f32_to_bf16_bits((x + gptq_ref.bf16_bits_to_f32(add_bits)).astype(np.float32)))
    var = np.float32((x.astype(np.float64) ** 2).mean(axis=-1, keepdims=True))
    r = (np.float32(1.0) / np.sqrt(var + np.float32(eps), dtype=np.float32)).astype(np.float32)
    w1 = (np.float32(1.0) + gptq_ref.bf16_bits_to_f32(weight_bits)).astype(np.float32)
    out = ((x * r).astype(np.float32) * w1).astype(np.float32)
    return gptq_ref.f32_to_bf16_bits(x), gptq_ref.f32_to_bf16_bits(out)


# --------------------------------------------------------------------------- hidden-residual predictor
def _bf16r(v: np.ndarray) -> np.ndarray:
    return gptq_ref.bf16_bits_to_f32(gptq_ref.f32_to_bf16_bits(np.asarray(v, dtype=np.float32)))


def hidden_residual_ref(h_bits: np.ndarray, p: dict, layer_ids: np.ndarray, *, top_k: int,
                        prior: np.ndarray | None = None, scale: float = 1.0,
                        scale_per_example: np.ndarray | None = None, ln_eps: float = 1e-5):
    """HiddenResidualExpertPredictor.forward (training/hidden_residual.py:44-106) with bf16
    activations between its Linear layers, the residual combination prior + scale * residual
    (scripts/train_hidden_residual_predictor_smoke.py:446) and the stable top-k per row.

    p: enc_w / ln_w / ln_b / layer_emb / delta_emb / cls_w as bf16 bits, enc_b / cls_b fp32.
    Steps (fp32 unless rounded): z = bf16(canonical(x, W_enc) + b_enc); a = bf16(silu(z));
    s = bf16(LayerNorm(a) * ln_w + ln_b) with float64 statistics rounded to fp32;
    c_d = bf16(bf16(s + E_layer[l]) + E_delta[d]); g_d = bf16(silu(c_d));
    r = canonical(g, W_cls) + b_cls. Returns (ids [N, F, k], out [N, F, E], residual [N, F, E])."""
    h = gptq_ref.bf16_bits_to_f32(h_bits)
    N = h.shape[0]
    enc_w = gptq_ref.bf16_bits_to_f32(p["enc_w"])
    W = enc_w.shape[0]
    z = _bf16r(canonical_dot_rows(h, enc_w) + p["enc_b"].astype(np.float32)[None, :])
    a = _bf16r(z / (np.float32(1.0) + np.exp(-z)))
    mean = a.astype(np.float64).mean(axis=1, keepdims=True).astype(np.float32)
    var = ((a - mean).astype(np.float64) ** 2).mean(axis=1, keepdims=True).astype(np.float32)
    rstd = (np.float32(1.0) / np.sqrt(var + np.float32(ln_eps))).astype(np.float32)
    s = _bf16r(((a - mean) * rstd).astype(np.float32) * gptq_ref.bf16_bits_to_f32(p["ln_w"])[None, :]
               + gptq_ref.bf16_bits_to_f32(p["ln_b"])[None, :])
    lemb = gptq_ref.bf16_bits_to_f32(p["layer_emb"])
    ok = (layer_ids >= 0) & (layer_ids < lemb.shape[0])
    le = np.where(ok[:, None], lemb[np.clip(layer_ids, 0, lemb.shape[0] - 1)], np.float32(0.0))
    sl = _bf16r(s + le)
    demb = gptq_ref.bf16_bits_to_f32(p["delta_emb"])
    F = demb.shape[0]
    c = _bf16r(sl[:, None, :] + demb[None, :, :])
    g = _bf16r(c / (np.float32(1.0) + np.exp(-c)))
    cls_w = gptq_ref.bf16_bits_to_f32(p["cls_w"])
    E = cls_w.shape[0]
    r = (canonical_dot_rows(g.reshape(N * F, W), cls_w) + p["cls_b"].astype(np.float32)[None, :])
    r = r.astype(np.float32).reshape(N, F, E)
    sc = (np.asarray(scale_per_example, dtype=np.float32)[:, None, None] if scale_per_example is not None
          else np.float32(scale))
    base = np.zeros_like(r) if prior is None else prior.astype(np.float32)
    out = (base + (sc * r).astype(np.float32)).astype(np.float32)
    ids = stable_topk(out.reshape(N * F, E), top_k).reshape(N, F, top_k)
    return ids, out, r
