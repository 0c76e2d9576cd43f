"""Seeded synthetic Qwen3.6-35B-A3B-shaped GPTQ-int4 MoE layers.

Shapes: hidden 2048, 256 experts, moe_intermediate 512, top-8, group 128
(configs/model/qwen3_6_35b_a3b_gptq_vllm_text_config/config.json:14, 66, 70-72, 77-129).
Distributions: qweight / qzeros uniform over all 32-bit patterns (every nibble U{0..15}),
fp16 scales U[0.002, 0.02], router weight bf16 N(0, 0.02), activations bf16 N(0, 1).
Seeds: weights 1000 + layer, router 2000 + layer, expert permutation 3000 + layer, x 7.

Generation uses a torch.Generator on the device the tensors are made on; small parity cases
are made on the CPU (device-independent bytes) and copied.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from mtp_amd.weights import GptqStack, MoeExperts

HIDDEN = 2048
NUM_EXPERTS = 256
INTERMEDIATE = 512
TOP_K = 8
GROUP = 128
ZIPF_S = 1.1
# Logit bias scale: b[perm[i]] = ZIPF_TAU * ln(p_i), p_i ~ i^-1.1, calibrated so the realised
# per-expert top-8 selection frequencies over 65536 tokens best fit Zipf(1.1)
# (mtp_amd/calibrate_zipf.py writes this value).
ZIPF_TAU = 0.5


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def _rand_u32_as_i32(shape, gen, device) -> torch.Tensor:
    # all 2^32 bit patterns equally likely; stored as int32 (two's complement)
    v = torch.randint(0, 1 << 32, shape, dtype=torch.int64, generator=gen, device=device)
    return (v - (1 << 31)).to(torch.int32) ^ torch.tensor(-(1 << 31), dtype=torch.int32, device=device)


def make_projection(num: int, k: int, n: int, gen, device, group: int = GROUP) -> GptqStack:
    qweight = _rand_u32_as_i32((num, k // 8, n), gen, device)
    qzeros = _rand_u32_as_i32((num, k // group, n // 8), gen, device)
    scales = torch.empty((num, k // group, n), dtype=torch.float32, device=device)
    scales.uniform_(0.002, 0.02, generator=gen)
    return GptqStack(qweight, qzeros, scales.to(torch.float16), None)


def make_experts(num_experts: int = NUM_EXPERTS, hidden: int = HIDDEN,
                 intermediate: int = INTERMEDIATE, *, seed: int = 1000, device="cpu",
                 group: int = GROUP) -> MoeExperts:
    gen = _gen(seed, device)
    gate = make_projection(num_experts, hidden, intermediate, gen, device, group)
    up = make_projection(num_experts, hidden, intermediate, gen, device, group)
    down = make_projection(num_experts, intermediate, hidden, gen, device, group)
    return MoeExperts(gate, up, down, group)


def make_router(num_experts: int = NUM_EXPERTS, hidden: int = HIDDEN, *, seed: int = 2000,
                device="cpu") -> torch.Tensor:
    gen = _gen(seed, device)
    w = torch.randn((num_experts, hidden), dtype=torch.float32, generator=gen, device=device) * 0.02
    return w.to(torch.bfloat16)


def make_shared_gate(hidden: int = HIDDEN, *, seed: int = 2500, device="cpu") -> torch.Tensor:
    gen = _gen(seed, device)
    return (torch.randn((hidden,), dtype=torch.float32, generator=gen, device=device) * 0.02).to(
        torch.bfloat16)


def make_tokens(T: int, hidden: int = HIDDEN, *, seed: int = 7, device="cpu") -> torch.Tensor:
    gen = _gen(seed, device)
    return torch.randn((T, hidden), dtype=torch.float32, generator=gen, device=device).to(
        torch.bfloat16)


def zipf_logit_bias(num_experts: int = NUM_EXPERTS, *, seed: int = 3000, tau: float = ZIPF_TAU,
                    s: float = ZIPF_S, device="cpu") -> torch.Tensor:
    """Per-layer router logit bias b[perm[i]] = tau * ln(p_i), p_i proportional to i^-s."""
    ranks = torch.arange(1, num_experts + 1, dtype=torch.float64)
    p = ranks.pow(-s)
    p = p / p.sum()
    perm = torch.randperm(num_experts, generator=_gen(seed, "cpu"))
    bias = torch.empty(num_experts, dtype=torch.float64)
    bias[perm] = tau * torch.log(p)
    return bias.to(torch.float32).to(device)


@dataclass
class SyntheticLayer:
    experts: MoeExperts
    router_w: torch.Tensor
    logit_bias: torch.Tensor | None
    shared: MoeExperts | None = None
    shared_gate_w: torch.Tensor | None = None


def make_layer(layer: int = 0, *, num_experts: int = NUM_EXPERTS, hidden: int = HIDDEN,
               intermediate: int = INTERMEDIATE, zipf: bool = False, shared: bool = False,
               device="cpu", group: int = GROUP) -> SyntheticLayer:
    experts = make_experts(num_experts, hidden, intermediate, seed=1000 + layer, device=device,
                           group=group)
    router = make_router(num_experts, hidden, seed=2000 + layer, device=device)
    bias = zipf_logit_bias(num_experts, seed=3000 + layer, device=device) if zipf else None
    sh = sg = None
    if shared:
        sh = make_experts(1, hidden, intermediate, seed=4000 + layer, device=device, group=group)
        sg = make_shared_gate(hidden, seed=2500 + layer, device=device)
    return SyntheticLayer(experts, router, bias, sh, sg)


def layer_to(layer: SyntheticLayer, device) -> SyntheticLayer:
    def mv(e: MoeExperts | None):
        if e is None:
            return None
        return MoeExperts(e.gate.to(device), e.up.to(device), e.down.to(device), e.group_size)
    return SyntheticLayer(mv(layer.experts), layer.router_w.to(device),
                          None if layer.logit_bias is None else layer.logit_bias.to(device),
                          mv(layer.shared),
                          None if layer.shared_gate_w is None else layer.shared_gate_w.to(device))


def expert_bytes(hidden: int = HIDDEN, intermediate: int = INTERMEDIATE, group: int = GROUP) -> int:
    """Packed qweight + fp16 scales + packed qzeros of one expert: 1 634 304 B at the default shape."""
    total = 0
    for k, n in ((hidden, intermediate), (hidden, intermediate), (intermediate, hidden)):
        total += (k // 8) * n * 4 + (k // group) * n * 2 + (k // group) * (n // 8) * 4
    return total


def prefill_flops(T: int, top_k: int = TOP_K, hidden: int = HIDDEN,
                  intermediate: int = INTERMEDIATE) -> int:
    """Useful (unpadded) expert FLOPs: 2*T*k*(H*2I + I*H)."""
    return 2 * T * top_k * (hidden * 2 * intermediate + intermediate * hidden)


assert expert_bytes() == 1_634_304
assert prefill_flops(2048) == 103_079_215_104
