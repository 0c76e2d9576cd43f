"""MoE block API: router_topk, moe_tokens and the fused layer forward.

Mirrors MtpExtraRunner.router_topk / moe_token / moe_tokens
(src/mtp_expert_prefetch/mtp/extra_tensors.py:341-356, 522-598) for the MoE part of the
layer: routed int4 experts plus an optional sigmoid-gated shared expert. Routing semantics are
vLLM's topk_softmax(renormalize=True) (src/mtp_expert_prefetch/tracing/vllm_router_trace.py:
4201-4225) with a stable tie rule, as the production path uses them.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from mtp_amd import ops
from mtp_amd.weights import MoeExperts


@dataclass(frozen=True)
class MoeRouterOutput:
    logits: torch.Tensor        # fp32 [..., E]
    topk_ids: torch.Tensor      # int32 [..., k]
    topk_weights: torch.Tensor  # fp32 [..., k]


class MoeBlock(torch.nn.Module):
    def __init__(self, experts: MoeExperts, router_weight: torch.Tensor, *,
                 shared_expert: MoeExperts | None = None,
                 shared_expert_gate_weight: torch.Tensor | None = None, top_k: int = 8,
                 logit_bias: torch.Tensor | None = None) -> None:
        super().__init__()
        experts.validate()
        if (shared_expert is None) != (shared_expert_gate_weight is None):
            raise ValueError("shared_expert and shared_expert_gate_weight must be given together")
        if shared_expert is not None:
            shared_expert.validate()
        self.experts = experts
        self.router_weight = router_weight.contiguous()
        self.shared_expert = shared_expert
        self.shared_expert_gate_weight = (None if shared_expert_gate_weight is None
                                          else shared_expert_gate_weight.reshape(-1).contiguous())
        self.top_k = int(top_k)
        self.logit_bias = logit_bias
        self.hidden_size = experts.hidden_size
        self.num_experts = int(experts.num_experts)

    def _flat(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.hidden_size:
            raise ValueError(f"Expected hidden size {self.hidden_size}, got {x.shape[-1]}")
        return x.reshape(-1, self.hidden_size).to(torch.bfloat16).contiguous()

    def router_topk(self, hidden_states: torch.Tensor, *, top_k: int | None = None) -> MoeRouterOutput:
        k = self.top_k if top_k is None else int(top_k)
        if not 0 < k <= self.num_experts:
            raise ValueError(f"top_k must be in [1, {self.num_experts}], got {k}")
        flat = self._flat(hidden_states)
        ids, w, _, logits = ops.router_topk(flat, self.router_weight, k, logit_bias=self.logit_bias)
        lead = hidden_states.shape[:-1]
        return MoeRouterOutput(logits.reshape(*lead, -1), ids.reshape(*lead, k), w.reshape(*lead, k))

    def moe_tokens(self, hidden_states: torch.Tensor, expert_ids: torch.Tensor,
                   expert_weights: torch.Tensor) -> torch.Tensor:
        """Per-token routed experts (+ gated shared expert) with caller-given routing."""
        if hidden_states.ndim != 3:
            raise ValueError("hidden_states must be [batch, seq, hidden] for batched MoE, "
                             f"got {tuple(hidden_states.shape)}")
        if expert_ids.shape != expert_weights.shape:
            raise ValueError(f"expert_ids and expert_weights must have same shape; "
                             f"got {tuple(expert_ids.shape)} and {tuple(expert_weights.shape)}")
        if expert_ids.shape[:2] != hidden_states.shape[:2]:
            raise ValueError("expert ids/weights must share [batch, seq] with hidden_states; "
                             f"got {tuple(expert_ids.shape)} and {tuple(hidden_states.shape)}")
        flat = self._flat(hidden_states)
        T = flat.shape[0]
        k = math.prod(expert_ids.shape[2:])  # ids per token (the reference's reshape(T, -1))
        ids = expert_ids.reshape(T, k).to(device=flat.device, dtype=torch.int32).contiguous()
        if bool(((ids < 0) | (ids >= self.num_experts)).any()):
            raise KeyError(f"expert ids must lie in [0, {self.num_experts})")
        w = expert_weights.reshape(T, k).to(device=flat.device, dtype=torch.float32).contiguous()
        out = ops.fused_experts(flat, ids, w, self.experts, shared=self.shared_expert,
                                shared_gate_w=self.shared_expert_gate_weight)
        return out.reshape(hidden_states.shape)

    def forward(self, hidden_states: torch.Tensor, *, path: str = "auto",
                return_routing: bool = False):
        """Router + routed experts (+ shared expert) in one stream-ordered call chain."""
        flat = self._flat(hidden_states)
        res = ops.moe_layer(flat, self.router_weight, self.experts, top_k=self.top_k,
                            logit_bias=self.logit_bias, shared=self.shared_expert,
                            shared_gate_w=self.shared_expert_gate_weight, path=path,
                            return_routing=return_routing)
        if return_routing:
            out, ids, w = res
            return out.reshape(hidden_states.shape), ids, w
        return res.reshape(hidden_states.shape)
