"""Device containers for GPTQ-int4 expert stacks in the reference's repacked layout.

Layout (src/mtp_expert_prefetch/repack/qwen3_moe_gptq.py:142-198, store.py:126-137):
  experts.{gate_proj,up_proj,down_proj}.{qweight,qzeros,scales,g_idx} stacked over experts,
  qweight int32 [E, K/8, N], qzeros int32 [E, K/G, N/8], scales fp16 [E, K/G, N],
  g_idx int32 [E, K] (g_idx[k] = k // G for desc_act=false checkpoints).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from mtp_amd import _lib

PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
KINDS = ("qweight", "qzeros", "scales", "g_idx")


@dataclass
class GptqStack:
    """One projection stacked over experts (or over the slots of an HBM pool)."""

    qweight: torch.Tensor
    qzeros: torch.Tensor
    scales: torch.Tensor
    g_idx: torch.Tensor | None = None

    @property
    def num_rows(self) -> int:
        return int(self.qweight.shape[0])

    @property
    def in_features(self) -> int:
        return int(self.qweight.shape[1]) * 8

    @property
    def out_features(self) -> int:
        return int(self.qweight.shape[2])

    def validate(self, group_size: int, row_stride_bytes: int = 0) -> None:
        """Check dtypes and shapes. row_stride_bytes > 0: the rows are blobs of a slot pool, so
        each tensor's rows are contiguous and row r starts row_stride_bytes after row r - 1."""
        for name in ("qweight", "qzeros", "scales"):
            t = getattr(self, name)
            if not isinstance(t, torch.Tensor):
                raise TypeError(f"{name} must be a torch.Tensor")
            if t.ndim != 3:
                raise ValueError(f"{name} must be 3D [E, ...], got {tuple(t.shape)}")
            if row_stride_bytes:
                if not t[0].is_contiguous() or t.stride(0) * t.element_size() != row_stride_bytes:
                    raise ValueError(f"{name} rows must be contiguous and {row_stride_bytes} B apart")
            elif not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous")
        if self.qweight.dtype != torch.int32 or self.qzeros.dtype != torch.int32:
            raise TypeError("qweight and qzeros must be int32")
        if self.scales.dtype != torch.float16:
            raise TypeError(f"scales must be float16, got {self.scales.dtype}")
        e, k8, n = self.qweight.shape
        k = k8 * 8
        if k % group_size != 0:
            raise ValueError(f"in_features={k} is not a multiple of group_size={group_size}")
        ng = k // group_size
        if tuple(self.scales.shape) != (e, ng, n):
            raise ValueError(f"scales is {tuple(self.scales.shape)}, expected {(e, ng, n)}")
        if tuple(self.qzeros.shape) != (e, ng, n // 8):
            raise ValueError(f"qzeros is {tuple(self.qzeros.shape)}, expected {(e, ng, n // 8)}")
        if self.g_idx is not None:
            expected = torch.arange(k, dtype=torch.int32, device=self.g_idx.device) // group_size
            g = self.g_idx.reshape(-1, k)
            if not bool((g == expected).all()):
                raise NotImplementedError(
                    "the fused W4A16 kernels need g_idx[k] == k // group_size (desc_act=false); "
                    "use dequantize_gptq_projection for other g_idx orders")

    def struct(self) -> _lib.GptqProj:
        return _lib.GptqProj(self.qweight.data_ptr(), self.qzeros.data_ptr(), self.scales.data_ptr())

    def to(self, device) -> "GptqStack":
        return GptqStack(self.qweight.to(device), self.qzeros.to(device), self.scales.to(device),
                         None if self.g_idx is None else self.g_idx.to(device))


@dataclass
class MoeExperts:
    """gate/up/down int4 stacks of one layer, plus an optional expert -> row map."""

    gate: GptqStack
    up: GptqStack
    down: GptqStack
    group_size: int = 128
    expert_row: torch.Tensor | None = None  # int32 [num_experts] rows of the stacks
    num_experts: int | None = None           # logical expert count (defaults to stack rows)
    expert_stride_bytes: int = 0             # > 0: rows are blobs of a slot pool, this far apart

    def __post_init__(self) -> None:
        if self.num_experts is None:
            self.num_experts = (int(self.expert_row.numel()) if self.expert_row is not None
                                else self.gate.num_rows)
        self._validated = False

    @property
    def hidden_size(self) -> int:
        return self.gate.in_features

    @property
    def intermediate_size(self) -> int:
        return self.gate.out_features

    @property
    def device(self) -> torch.device:
        return self.gate.qweight.device

    def validate(self) -> None:
        if self._validated:
            return
        for p in (self.gate, self.up, self.down):
            p.validate(self.group_size, self.expert_stride_bytes)
        if self.expert_stride_bytes and self.expert_row is None:
            raise ValueError("a slot pool (expert_stride_bytes > 0) needs expert_row")
        h, i = self.hidden_size, self.intermediate_size
        if self.up.in_features != h or self.up.out_features != i:
            raise ValueError("gate_proj and up_proj shapes must match")
        if self.down.in_features != i or self.down.out_features != h:
            raise ValueError(f"down_proj must map {i} -> {h}")
        if self.expert_row is not None:
            if self.expert_row.dtype != torch.int32 or self.expert_row.device != self.device:
                raise TypeError("expert_row must be int32 on the weights' device")
        self._validated = True

    def struct(self) -> _lib.ExpertSet:
        self.validate()
        return _lib.ExpertSet(
            self.gate.struct(), self.up.struct(), self.down.struct(),
            0 if self.expert_row is None else self.expert_row.data_ptr(),
            int(self.num_experts), self.hidden_size, self.intermediate_size, int(self.group_size),
            int(self.expert_stride_bytes))

    def nbytes_per_expert(self) -> int:
        """Packed qweight + fp16 scales + packed qzeros of one expert (g_idx excluded)."""
        total = 0
        for p in (self.gate, self.up, self.down):
            for t in (p.qweight, p.qzeros, p.scales):
                total += t[0].numel() * t.element_size()
        return total

    @classmethod
    def from_tensors(cls, tensors: dict[str, torch.Tensor], *, group_size: int = 128,
                     prefix: str = "experts.") -> "MoeExperts":
        """Build from the repacked store's keys 'experts.{proj}.{kind}'."""
        stacks = {}
        for proj in PROJECTIONS:
            stacks[proj] = GptqStack(
                tensors[f"{prefix}{proj}.qweight"], tensors[f"{prefix}{proj}.qzeros"],
                tensors[f"{prefix}{proj}.scales"], tensors.get(f"{prefix}{proj}.g_idx"))
        return cls(stacks["gate_proj"], stacks["up_proj"], stacks["down_proj"], group_size)
