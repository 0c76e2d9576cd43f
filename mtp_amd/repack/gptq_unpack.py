"""The reference's GPTQ expert API, backed by the MI355X W4A16 kernels.

Mirrors src/mtp_expert_prefetch/repack/gptq_unpack.py (names, argument meaning, error
types and messages), with one design change: experts stay int4 on the device and run through
the fused HIP kernels instead of being dequantised to dense bf16 at load time.

  GptqProjectionTensors        :12-16
  resolve_torch_dtype          :44-51
  unpack_cols / unpack_rows    :54-85   (format helpers on torch tensors; not on the hot path)
  dequantize_gptq_projection   :88-131  (HIP dequant kernel; bit-exact)
  synthesize_g_idx             :134-148
  load_repacked_projection_tensors / dequantize_repacked_projection :151-184
  apply_dequantized_projection :187-188
  load_single_expert_weights   :191-228 (dense dequantised weights, via the HIP kernel)
  SingleExpertMlp              :231-256 (int4 expert, fused W1/W2 kernels)
  TopKExpertMlp                :259-327 (int4 experts, fused W1/W2 kernels)
  load_single_expert_mlp / load_topk_expert_mlp :330-371
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from mtp_amd import ops
from mtp_amd.repack.store import RepackedMoeExpertStore
from mtp_amd.weights import GptqStack, MoeExperts


@dataclass(frozen=True)
class GptqProjectionTensors:
    qweight: torch.Tensor
    qzeros: torch.Tensor
    scales: torch.Tensor
    g_idx: torch.Tensor


@dataclass(frozen=True)
class SingleExpertWeights:
    """Dense Linear-orientation weights of one expert (gate/up [I, H], down [H, I])."""

    gate_proj: torch.Tensor
    up_proj: torch.Tensor
    down_proj: torch.Tensor

    @property
    def hidden_size(self) -> int:
        return int(self.gate_proj.shape[1])

    @property
    def intermediate_size(self) -> int:
        return int(self.gate_proj.shape[0])


@dataclass(frozen=True)
class QuantizedExpertWeights:
    """int4 GPTQ tensors of one expert; the form the fused kernels consume."""

    gate_proj: GptqProjectionTensors
    up_proj: GptqProjectionTensors
    down_proj: GptqProjectionTensors
    group_size: int = 128

    @property
    def hidden_size(self) -> int:
        return int(self.gate_proj.qweight.shape[0]) * 8

    @property
    def intermediate_size(self) -> int:
        return int(self.gate_proj.qweight.shape[1])


DTYPE_NAMES = {
    "float16": torch.float16,
    "fp16": torch.float16,
    "bfloat16": torch.bfloat16,
    "bf16": torch.bfloat16,
    "float32": torch.float32,
    "fp32": torch.float32,
}


def resolve_torch_dtype(dtype: str | torch.dtype) -> torch.dtype:
    if isinstance(dtype, torch.dtype):
        return dtype
    try:
        return DTYPE_NAMES[dtype.lower()]
    except KeyError as exc:
        msg = f"Unsupported dtype {dtype!r}; expected one of {sorted(DTYPE_NAMES)}"
        raise ValueError(msg) from exc


def _validate_bits(bits: int) -> None:
    if bits not in (2, 4, 8):
        msg = f"This unpacker supports 2/4/8-bit GPTQ rows/cols; got bits={bits}"
        raise ValueError(msg)


def _unpack(packed: torch.Tensor, bits: int, along_rows: bool) -> torch.Tensor:
    _validate_bits(bits)
    pack_bits = packed.element_size() * 8
    factor = pack_bits // bits
    mask = (1 << bits) - 1
    u = packed.to(torch.int64) & ((1 << pack_bits) - 1)
    shifts = torch.arange(factor, device=packed.device, dtype=torch.int64) * bits
    rows, cols = packed.shape
    if along_rows:  # out[factor*r + j, c] = field j of packed[r, c]
        v = (u[:, None, :] >> shifts[None, :, None]) & mask
        return v.reshape(rows * factor, cols).to(torch.int32)
    v = (u[:, :, None] >> shifts[None, None, :]) & mask  # out[r, factor*c + j]
    return v.reshape(rows, cols * factor).to(torch.int32)


def unpack_cols(packed: torch.Tensor, *, bits: int = 4) -> torch.Tensor:
    """Unpack GPTQ int32 values packed along the column dimension."""
    return _unpack(packed, bits, along_rows=False)


def unpack_rows(packed: torch.Tensor, *, bits: int = 4) -> torch.Tensor:
    """Unpack GPTQ int32 values packed along the input-row dimension."""
    return _unpack(packed, bits, along_rows=True)


def _validate_projection_tensors(tensors: GptqProjectionTensors) -> None:
    for name in ("qweight", "qzeros", "scales", "g_idx"):
        if not isinstance(getattr(tensors, name), torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
    if tensors.qweight.ndim != 2:
        raise ValueError(f"qweight must be 2D, got {tuple(tensors.qweight.shape)}")
    if tensors.qzeros.ndim != 2:
        raise ValueError(f"qzeros must be 2D, got {tuple(tensors.qzeros.shape)}")
    if tensors.scales.ndim != 2:
        raise ValueError(f"scales must be 2D, got {tuple(tensors.scales.shape)}")
    if tensors.g_idx.ndim != 1:
        raise ValueError(f"g_idx must be 1D, got {tuple(tensors.g_idx.shape)}")


def dequantize_gptq_projection(
    tensors: GptqProjectionTensors,
    *,
    bits: int = 4,
    dtype: str | torch.dtype = torch.bfloat16,
    linear_weight: bool = True,
) -> torch.Tensor:
    """Dequantize one GPTQ projection on the GPU (bit-exact with the reference formula).

    Returns PyTorch Linear orientation `[out_features, in_features]` by default.
    Set `linear_weight=False` to get GPTQ internal orientation `[in_features, out_features]`.
    """
    _validate_projection_tensors(tensors)
    _validate_bits(bits)
    if bits != 4:
        raise NotImplementedError("the HIP dequant kernel implements the 4-bit GPTQ layout")
    target_dtype = resolve_torch_dtype(dtype)
    rows_in = int(tensors.qweight.shape[0]) * 8
    cols_out = int(tensors.qweight.shape[1])
    g_idx = tensors.g_idx.to(torch.long)
    if rows_in != g_idx.numel():
        msg = f"qweight expands to {rows_in} input rows, but g_idx has {g_idx.numel()}"
        raise ValueError(msg)
    if cols_out != tensors.scales.shape[1]:
        msg = (f"qweight expands to {cols_out} output columns, "
               f"but scales has {tensors.scales.shape[1]}")
        raise ValueError(msg)
    zeros_shape = (int(tensors.qzeros.shape[0]), int(tensors.qzeros.shape[1]) * 8)
    if zeros_shape != tuple(tensors.scales.shape):
        msg = f"qzeros expands to {zeros_shape}, but scales is {tuple(tensors.scales.shape)}"
        raise ValueError(msg)
    num_groups = int(tensors.scales.shape[0])
    if int(g_idx.min()) < 0 or int(g_idx.max()) >= num_groups:
        msg = (f"g_idx out of range: min={int(g_idx.min())}, max={int(g_idx.max())}, "
               f"num_groups={num_groups}")
        raise ValueError(msg)
    group_size = rows_in // num_groups
    return ops.dequantize(tensors.qweight.contiguous(), tensors.qzeros.contiguous(),
                          tensors.scales.to(torch.float16).contiguous(),
                          tensors.g_idx.to(torch.int32).contiguous(), group_size=group_size,
                          linear_weight=linear_weight, dtype=target_dtype)


def synthesize_g_idx(qweight: torch.Tensor, *, bits: int = 4, group_size: int = 128) -> torch.Tensor:
    """Create GPTQ group indices for checkpoints that omit static `g_idx`."""
    _validate_bits(bits)
    if qweight.ndim != 2:
        raise ValueError(f"qweight must be 2D, got {tuple(qweight.shape)}")
    if group_size <= 0:
        raise ValueError(f"group_size must be positive, got {group_size}")
    pack_factor = qweight.element_size() * 8 // bits
    in_features = int(qweight.shape[0]) * pack_factor
    return torch.arange(in_features, dtype=torch.int32, device=qweight.device) // int(group_size)


def load_repacked_projection_tensors(store: RepackedMoeExpertStore, *, layer: int, expert: int,
                                     projection: str, device: str | torch.device = "cpu"
                                     ) -> GptqProjectionTensors:
    return GptqProjectionTensors(
        qweight=store.get_expert_tensor(layer, expert, projection, "qweight").to(device=device),
        qzeros=store.get_expert_tensor(layer, expert, projection, "qzeros").to(device=device),
        scales=store.get_expert_tensor(layer, expert, projection, "scales").to(device=device),
        g_idx=store.get_expert_tensor(layer, expert, projection, "g_idx").to(device=device),
    )


def dequantize_repacked_projection(store: RepackedMoeExpertStore, *, layer: int, expert: int,
                                   projection: str, bits: int = 4,
                                   dtype: str | torch.dtype = torch.bfloat16,
                                   device: str | torch.device = "cuda") -> torch.Tensor:
    tensors = load_repacked_projection_tensors(store, layer=layer, expert=expert,
                                               projection=projection, device=device)
    return dequantize_gptq_projection(tensors, bits=bits, dtype=dtype)


def apply_dequantized_projection(input_tensor: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    return F.linear(input_tensor, weight)


def load_single_expert_weights(store: RepackedMoeExpertStore, *, layer: int, expert: int,
                               bits: int = 4, dtype: str | torch.dtype = torch.bfloat16,
                               device: str | torch.device = "cuda") -> SingleExpertWeights:
    """Dense dequantised weights of one expert (HIP dequant kernel)."""
    projs = {p: dequantize_repacked_projection(store, layer=layer, expert=expert, projection=p,
                                               bits=bits, dtype=dtype, device=device)
             for p in ("gate_proj", "up_proj", "down_proj")}
    weights = SingleExpertWeights(projs["gate_proj"], projs["up_proj"], projs["down_proj"])
    _validate_single_expert_weights(weights)
    return weights


def _stack(experts: list[QuantizedExpertWeights], attr: str) -> GptqStack:
    ps = [getattr(e, attr) for e in experts]
    return GptqStack(torch.stack([p.qweight for p in ps]).contiguous(),
                     torch.stack([p.qzeros for p in ps]).contiguous(),
                     torch.stack([p.scales.to(torch.float16) for p in ps]).contiguous(),
                     torch.stack([p.g_idx.to(torch.int32) for p in ps]).contiguous())


def _as_quantized(weights) -> QuantizedExpertWeights:
    if isinstance(weights, QuantizedExpertWeights):
        return weights
    raise TypeError(
        "the W4A16 expert kernels take int4 GPTQ tensors (QuantizedExpertWeights); dense "
        "SingleExpertWeights have no int4 form to run")


class SingleExpertMlp(torch.nn.Module):
    """y = W_down (silu(W_gate x) * (W_up x)) on int4 weights (gptq_unpack.py:231-256)."""

    def __init__(self, weights: QuantizedExpertWeights) -> None:
        super().__init__()
        q = _as_quantized(weights)
        self.quantized = q
        self.stack = MoeExperts(_stack([q], "gate_proj"), _stack([q], "up_proj"),
                                _stack([q], "down_proj"), q.group_size)
        self.stack.validate()

    @property
    def hidden_size(self) -> int:
        return self.stack.hidden_size

    @property
    def intermediate_size(self) -> int:
        return self.stack.intermediate_size

    def forward(self, input_tensor: torch.Tensor) -> torch.Tensor:
        if input_tensor.shape[-1] != self.hidden_size:
            msg = f"Expected input last dim {self.hidden_size}, got {input_tensor.shape[-1]}"
            raise ValueError(msg)
        x = input_tensor.reshape(-1, self.hidden_size).contiguous()
        T = x.shape[0]
        ids = torch.zeros(T, 1, dtype=torch.int32, device=x.device)
        w = torch.ones(T, 1, dtype=torch.float32, device=x.device)
        out = ops.fused_experts(x, ids, w, self.stack)
        return out.reshape(input_tensor.shape)


class TopKExpertMlp(torch.nn.Module):
    """sum_i w_i * expert_{id_i}(x) over one shared expert set (gptq_unpack.py:259-327)."""

    def __init__(self, experts: dict[int, SingleExpertMlp | QuantizedExpertWeights]) -> None:
        super().__init__()
        if not experts:
            msg = "TopKExpertMlp requires at least one expert"
            raise ValueError(msg)
        quant = {int(k): (v.quantized if isinstance(v, SingleExpertMlp) else _as_quantized(v))
                 for k, v in experts.items()}
        hidden_sizes = {q.hidden_size for q in quant.values()}
        intermediate_sizes = {q.intermediate_size for q in quant.values()}
        if len(hidden_sizes) != 1 or len(intermediate_sizes) != 1:
            msg = (f"All experts must share dimensions; got hidden={hidden_sizes}, "
                   f"intermediate={intermediate_sizes}")
            raise ValueError(msg)
        self._ids = tuple(sorted(quant))
        ordered = [quant[i] for i in self._ids]
        self.stack = MoeExperts(_stack(ordered, "gate_proj"), _stack(ordered, "up_proj"),
                                _stack(ordered, "down_proj"), ordered[0].group_size)
        self.stack.validate()
        self._row = {eid: row for row, eid in enumerate(self._ids)}

    @property
    def loaded_expert_ids(self) -> tuple[int, ...]:
        return self._ids

    @property
    def hidden_size(self) -> int:
        return self.stack.hidden_size

    @property
    def intermediate_size(self) -> int:
        return self.stack.intermediate_size

    def forward(self, input_tensor: torch.Tensor, expert_ids: torch.Tensor,
                expert_weights: torch.Tensor) -> torch.Tensor:
        if input_tensor.shape[-1] != self.hidden_size:
            msg = f"Expected input last dim {self.hidden_size}, got {input_tensor.shape[-1]}"
            raise ValueError(msg)
        if expert_ids.ndim != 1:
            msg = f"expert_ids must be 1D for this smoke path, got {tuple(expert_ids.shape)}"
            raise ValueError(msg)
        if expert_weights.ndim != 1:
            msg = f"expert_weights must be 1D for this smoke path, got {tuple(expert_weights.shape)}"
            raise ValueError(msg)
        if expert_ids.shape != expert_weights.shape:
            msg = (f"expert_ids and expert_weights must have same shape; "
                   f"got {tuple(expert_ids.shape)} and {tuple(expert_weights.shape)}")
            raise ValueError(msg)
        rows = []
        for expert_id in expert_ids.to(device="cpu", dtype=torch.long).tolist():
            if int(expert_id) not in self._row:
                msg = f"Expert {expert_id} is not loaded; loaded={self.loaded_expert_ids}"
                raise KeyError(msg)
            rows.append(self._row[int(expert_id)])
        x = input_tensor.reshape(-1, self.hidden_size).contiguous()
        T, k = x.shape[0], len(rows)
        dev = x.device
        ids = torch.tensor(rows, dtype=torch.int32, device=dev).expand(T, k).contiguous()
        # the reference casts the routing weights to the input dtype before use (:319)
        w = expert_weights.to(device=dev, dtype=input_tensor.dtype).to(torch.float32)
        w = w.expand(T, k).contiguous()
        out = ops.fused_experts(x, ids, w, self.stack)
        return out.reshape(input_tensor.shape)


def load_quantized_expert(store: RepackedMoeExpertStore, *, layer: int, expert: int,
                          device: str | torch.device = "cuda") -> QuantizedExpertWeights:
    projs = {p: load_repacked_projection_tensors(store, layer=layer, expert=expert, projection=p,
                                                 device=device)
             for p in ("gate_proj", "up_proj", "down_proj")}
    group = int(projs["gate_proj"].qweight.shape[0]) * 8 // int(projs["gate_proj"].scales.shape[0])
    return QuantizedExpertWeights(projs["gate_proj"], projs["up_proj"], projs["down_proj"], group)


def _check_bits_dtype(bits: int, dtype) -> None:
    _validate_bits(bits)
    if bits != 4:
        raise NotImplementedError("the fused expert kernels implement 4-bit GPTQ")
    if resolve_torch_dtype(dtype) != torch.bfloat16:
        raise NotImplementedError("the fused expert kernels compute with bf16 activations")


def load_single_expert_mlp(store: RepackedMoeExpertStore, *, layer: int, expert: int,
                           bits: int = 4, dtype: str | torch.dtype = torch.bfloat16,
                           device: str | torch.device = "cuda") -> SingleExpertMlp:
    _check_bits_dtype(bits, dtype)
    return SingleExpertMlp(load_quantized_expert(store, layer=layer, expert=expert, device=device))


def load_topk_expert_mlp(store: RepackedMoeExpertStore, *, layer: int,
                         expert_ids: list[int] | tuple[int, ...], bits: int = 4,
                         dtype: str | torch.dtype = torch.bfloat16,
                         device: str | torch.device = "cuda") -> TopKExpertMlp:
    _check_bits_dtype(bits, dtype)
    unique_expert_ids = tuple(dict.fromkeys(int(expert_id) for expert_id in expert_ids))
    experts = {eid: load_quantized_expert(store, layer=layer, expert=eid, device=device)
               for eid in unique_expert_ids}
    return TopKExpertMlp(experts)


def _validate_single_expert_weights(weights: SingleExpertWeights) -> None:
    gate_shape = tuple(weights.gate_proj.shape)
    up_shape = tuple(weights.up_proj.shape)
    down_shape = tuple(weights.down_proj.shape)
    if weights.gate_proj.ndim != 2 or weights.up_proj.ndim != 2 or weights.down_proj.ndim != 2:
        msg = f"SingleExpertMlp weights must be 2D; got gate={gate_shape}, up={up_shape}, down={down_shape}"
        raise ValueError(msg)
    if gate_shape != up_shape:
        msg = f"gate_proj and up_proj shapes must match; got gate={gate_shape}, up={up_shape}"
        raise ValueError(msg)
    if down_shape != (gate_shape[1], gate_shape[0]):
        msg = (f"down_proj must have shape [hidden, intermediate]; "
               f"got down={down_shape}, gate={gate_shape}")
        raise ValueError(msg)
