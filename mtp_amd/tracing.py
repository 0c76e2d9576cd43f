"""Router-trace payloads as the reference's trace smoke harness reads them.

The drop-in counterpart of src/mtp_expert_prefetch/tracing/router_trace_bridge.py (:15-228) for
scripts/smoke_trace_topk_expert_mlp.py (:60-137): a payload is a dict saved with torch.save,

* ``router_topk``: {router module name: [one entry per call: int ids [B, T, k], [T, k] or [k]]}
* ``router_scores`` (optional): the same structure with the scores of those ids,
* ``last_hidden_state`` (optional): [B, T, H] or [T, H],

and ``select_router_topk`` turns one (module, call, batch, token) of it into the expert ids and
routing weights that ``TopKExpertMlp`` takes. Names, fields, index rules and exception types
follow the reference. One difference: payloads are loaded with ``torch.load(weights_only=True)``,
so a file that holds anything beyond tensors and plain containers is refused (the reference
unpickles arbitrary objects).
"""

from __future__ import annotations

import json
import re
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import torch

__all__ = [
    "RouterTopKSelection",
    "load_trace_payload",
    "resolve_trace_sample",
    "select_router_topk",
    "select_trace_hidden_token",
    "resolve_router_module_name",
    "scores_to_router_weights",
]

# the router of decoder layer L: a module name ending in "layers.L.mlp.gate"
_ROUTER_OF_LAYER = r"(?:^|\.)layers\.{layer}\.mlp\.gate$"


@dataclass(frozen=True)
class RouterTopKSelection:
    module_name: str
    expert_ids: torch.Tensor       # int64 [k]
    expert_weights: torch.Tensor   # fp32 [k]
    raw_scores: torch.Tensor | None
    call_index: int
    batch_index: int | None
    token_index: int | None


def load_trace_payload(path: str | Path) -> dict[str, Any]:
    """The payload dict of one trace sample (tensors and plain containers only)."""
    p = Path(path).expanduser().resolve()
    payload = torch.load(p, map_location="cpu", weights_only=True)
    if not isinstance(payload, dict):
        raise TypeError(f"Expected trace payload dict in {p}, got {type(payload).__name__}")
    return payload


def resolve_trace_sample(*, sample_path: str | Path | None = None,
                         manifest_path: str | Path | None = None) -> Path:
    """An explicit sample path, else the first record of a JSON-lines manifest whose ``path``
    is relative to the manifest's directory."""
    if sample_path is not None:
        p = Path(sample_path).expanduser().resolve()
        if not p.exists():
            raise FileNotFoundError(f"Missing trace sample: {p}")
        return p
    if manifest_path is None:
        raise ValueError("Either sample_path or manifest_path is required.")
    m = Path(manifest_path).expanduser().resolve()
    if not m.exists():
        raise FileNotFoundError(f"Missing trace manifest: {m}")
    for line in m.read_text(encoding="utf-8").splitlines():
        if not line.strip():
            continue
        sample = m.parent / json.loads(line)["path"]
        if not sample.exists():
            raise FileNotFoundError(f"Manifest points to missing trace sample: {sample}")
        return sample.resolve()
    raise RuntimeError(f"Trace manifest has no sample records: {m}")


def _index(i: int, size: int, name: str) -> int:
    """Python-style index (negative counts from the end) checked against size."""
    if size <= 0:
        raise IndexError(f"Cannot index empty dimension for {name}.")
    j = i + size if i < 0 else i
    if not 0 <= j < size:
        raise IndexError(f"{name}={i} out of range for size {size}")
    return j


def _call(calls: Any, call_index: int, name: str) -> Any:
    if not isinstance(calls, list) or not calls:
        raise ValueError(f"{name} entry is empty or not a list.")
    return calls[_index(call_index, len(calls), "call_index")]


def _token_vector(t: torch.Tensor, batch_index: int, token_index: int) -> torch.Tensor:
    """The [k] vector of one token from [B, T, k], [T, k] or [k]."""
    if t.ndim == 3:
        return t[_index(batch_index, t.shape[0], "batch_index"),
                 _index(token_index, t.shape[1], "token_index")].contiguous()
    if t.ndim == 2:
        return t[_index(token_index, t.shape[0], "token_index")].contiguous()
    if t.ndim == 1:
        return t.contiguous()
    raise ValueError(f"Expected router top-k tensor with 1-3 dims, got {tuple(t.shape)}")


def resolve_router_module_name(router_topk: dict[str, Any], *, layer: int | None = None,
                               module_name: str | None = None) -> str:
    """An explicit module name, else the first name in sorted order (no layer), else the one
    router module of the layer."""
    if module_name is not None:
        if module_name not in router_topk:
            raise KeyError(f"Router module {module_name!r} not found. "
                           f"Available: {sorted(router_topk)[:16]}")
        return module_name
    names = sorted(router_topk)
    if layer is None:
        return names[0]
    rx = re.compile(_ROUTER_OF_LAYER.format(layer=layer))
    hits = [n for n in names if rx.search(n)]
    if not hits:  # looser: any "mlp.gate" module under "layers.L."
        hits = [n for n in names if f"layers.{layer}." in n and "mlp.gate" in n]
    if len(hits) != 1:
        raise KeyError(f"Expected exactly one router module for layer={layer}, found {hits}")
    return hits[0]


def scores_to_router_weights(scores: torch.Tensor, *, mode: str = "softmax") -> torch.Tensor:
    """Routing weights from the selected experts' scores: softmax, the scores themselves
    (raw / identity) or equal weights (uniform / equal); fp32."""
    if scores.ndim != 1:
        raise ValueError(f"scores must be 1D, got {tuple(scores.shape)}")
    m = mode.lower()
    if m == "softmax":
        return torch.softmax(scores.float(), dim=-1)
    if m in ("raw", "identity"):
        return scores.float()
    if m in ("uniform", "equal"):
        return torch.full(scores.shape, 1.0 / max(1, scores.numel()), dtype=torch.float32)
    raise ValueError(f"Unsupported scores_to_weights mode {mode!r}")


def select_router_topk(payload: dict[str, Any], *, layer: int | None = None,
                       module_name: str | None = None, call_index: int = 0,
                       batch_index: int = 0, token_index: int = 0, top_k: int | None = None,
                       scores_to_weights: str = "softmax") -> RouterTopKSelection:
    """One token's routed experts from a payload; weights from its scores when the payload has
    them, else equal weights."""
    topk = payload.get("router_topk")
    if not isinstance(topk, dict) or not topk:
        raise KeyError("Trace payload has no non-empty `router_topk` dict.")
    name = resolve_router_module_name(topk, layer=layer, module_name=module_name)
    ids = _token_vector(torch.as_tensor(_call(topk[name], call_index, "router_topk"),
                                        dtype=torch.long), batch_index, token_index)
    if top_k is not None:
        ids = ids[:top_k]
    raw = None
    scores = payload.get("router_scores")
    if isinstance(scores, dict) and name in scores:
        raw = _token_vector(torch.as_tensor(_call(scores[name], call_index, "router_scores"),
                                            dtype=torch.float32), batch_index, token_index)
        if top_k is not None:
            raw = raw[:top_k]
        weights = scores_to_router_weights(raw, mode=scores_to_weights)
    else:
        weights = torch.full(ids.shape, 1.0 / max(1, ids.numel()), dtype=torch.float32)
    return RouterTopKSelection(module_name=name, expert_ids=ids.to(torch.long),
                               expert_weights=weights.to(torch.float32), raw_scores=raw,
                               call_index=call_index, batch_index=batch_index,
                               token_index=token_index)


def select_trace_hidden_token(payload: dict[str, Any], *, batch_index: int = 0,
                              token_index: int = 0) -> torch.Tensor:
    """One token's hidden state, keeping the payload's rank: [1, 1, H] from [B, T, H], [1, H]
    from [T, H]."""
    h = payload.get("last_hidden_state")
    if not isinstance(h, torch.Tensor):
        raise KeyError("Trace payload has no `last_hidden_state` tensor.")
    if h.ndim == 3:
        b = _index(batch_index, h.shape[0], "batch_index")
        t = _index(token_index, h.shape[1], "token_index")
        return h[b:b + 1, t:t + 1, :].contiguous()
    if h.ndim == 2:
        t = _index(token_index, h.shape[0], "token_index")
        return h[t:t + 1, :].contiguous()
    raise ValueError(f"Unsupported last_hidden_state shape: {tuple(h.shape)}")
