"""AWQ int4 checkpoints on the W4A16 kernels: an exact repack into the GPTQ layout on the GPU.

Layouts (moe_awq_to_gptq_v1):
  "wna16"  vLLM's int4 fused-MoE layout the reference serves its AWQ checkpoint with
           (src/mtp_expert_prefetch/tracing/vllm_wna16_group_plan.py:394-470;
           configs/model/qwen3_6_35b_a3b_awq_4bit.yaml): qweight uint8 [E, N, K/2] (low nibble =
           even k), qzeros uint8 [E, N/2, K/G] (low nibble = even n) or None (zero 8), scales
           fp16 or bf16 [E, N, K/G].
  "awq"    the AutoAWQ GEMM checkpoint layout: qweight int32 [E, K, N/8], qzeros int32
           [E, K/G, N/8], both packed along N in the order [0, 2, 4, 6, 1, 3, 5, 7]; scales fp16
           [E, K/G, N].
The repacked stack dequantises to exactly the same (q - z) * s, so the layer computed on it is
the AWQ checkpoint's layer.
"""

from __future__ import annotations

import ctypes

import torch

from mtp_amd import _lib
from mtp_amd.weights import GptqStack, MoeExperts

LAYOUTS = {"wna16": 1, "awq": 2}


def _check(t: torch.Tensor, name: str, dtypes, shape) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype not in dtypes:
        raise TypeError(f"{name} must be one of {dtypes}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous ROCm device tensor")


def awq_to_gptq(qweight: torch.Tensor, qzeros: torch.Tensor | None, scales: torch.Tensor, *,
                layout: str, in_features: int, group_size: int) -> GptqStack:
    """Repack one projection stacked over experts into the GPTQ layout (qweight int32
    [E, K/8, N], qzeros int32 [E, K/G, N/8], scales fp16 [E, K/G, N]). Synchronises once to
    read the exactness flag and raises ValueError if a bf16 scale has no exact fp16 value."""
    lib = _lib.load()
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be one of {sorted(LAYOUTS)}")
    K, G = int(in_features), int(group_size)
    if K % G or K % 8:
        raise ValueError(f"in_features={K} must be a multiple of 8 and of group_size={G}")
    NG = K // G
    if layout == "wna16":
        E, N = int(qweight.shape[0]), int(qweight.shape[1])
        _check(qweight, "qweight", (torch.uint8,), (E, N, K // 2))
        if qzeros is not None:
            _check(qzeros, "qzeros", (torch.uint8,), (E, N // 2, NG))
        _check(scales, "scales", (torch.float16, torch.bfloat16), (E, N, NG))
    else:
        E, N = int(qweight.shape[0]), int(qweight.shape[2]) * 8
        _check(qweight, "qweight", (torch.int32,), (E, K, N // 8))
        if qzeros is None:
            raise ValueError("the AutoAWQ GEMM layout needs qzeros")
        _check(qzeros, "qzeros", (torch.int32,), (E, NG, N // 8))
        _check(scales, "scales", (torch.float16,), (E, NG, N))
    dev = qweight.device
    out = GptqStack(torch.empty(E, K // 8, N, dtype=torch.int32, device=dev),
                    torch.empty(E, NG, N // 8, dtype=torch.int32, device=dev),
                    torch.empty(E, NG, N, dtype=torch.float16, device=dev))
    status = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.check(lib.moe_awq_to_gptq_v1(
        LAYOUTS[layout], qweight.data_ptr(), None if qzeros is None else qzeros.data_ptr(),
        scales.data_ptr(), int(scales.dtype == torch.bfloat16), E, K, N, G,
        ctypes.byref(out.struct()), status.data_ptr(),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    if int(status.item()) != 0:
        raise ValueError("a bf16 scale has no exact fp16 value (|s| outside [2^-17, 65504]); the "
                         "int4 kernels take fp16 scales")
    return out


def load_awq_experts(gate, up, down, *, layout: str, hidden: int, intermediate: int,
                     group_size: int = 128) -> MoeExperts:
    """An AWQ expert set ((qweight, qzeros, scales) per projection, stacked over experts) as the
    kernels' MoeExperts: gate/up map hidden -> intermediate, down intermediate -> hidden."""
    stacks = [awq_to_gptq(*p, layout=layout, in_features=k, group_size=group_size)
              for p, k in ((gate, hidden), (up, hidden), (down, intermediate))]
    ex = MoeExperts(*stacks, group_size)
    ex.validate()
    return ex
