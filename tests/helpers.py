"""Shared test helpers: synthetic layers in the oracle's numpy format, comparisons."""

from __future__ import annotations

import numpy as np
import torch

from mtp_amd import synth
from mtp_amd.weights import MoeExperts

# Layer-output tolerance: max|out - ref| / max|ref| (bf16 output against the fp32-accumulated
# oracle). The target for this path is 1e-2.
LAYER_RTOL = 1e-2


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def experts_to_np(ex: MoeExperts) -> dict:
    d = {"group_size": ex.group_size}
    for name, st in (("gate_proj", ex.gate), ("up_proj", ex.up), ("down_proj", ex.down)):
        d[f"{name}.qweight"] = st.qweight.detach().cpu().numpy()
        d[f"{name}.qzeros"] = st.qzeros.detach().cpu().numpy()
        d[f"{name}.scales"] = f16_bits(st.scales)
    return d


def small_layer(layer: int = 0, *, E: int = 16, H: int = 512, I: int = 256, zipf: bool = False,
                shared: bool = False) -> synth.SyntheticLayer:
    return synth.make_layer(layer, num_experts=E, hidden=H, intermediate=I, zipf=zipf,
                            shared=shared, device="cpu")


def to_gpu(layer: synth.SyntheticLayer) -> synth.SyntheticLayer:
    return synth.layer_to(layer, "cuda")
