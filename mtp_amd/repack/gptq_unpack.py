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
  SingleExpertMlp              :231-256 (int4 expert as non-persistent buffers, fused W1/W2
                                         kernels; gate_proj/up_proj/down_proj dequantised on use)
  TopKExpertMlp                :259-327 (int4 experts stacked as buffers, fused W1/W2 kernels)
  load_single_expert_mlp / load_topk_expert_mlp :330-371 (bf16, fp16 and fp32 dtypes)

Activations enter the kernels as bf16: an fp16 or fp32 input is rounded to bf16, the expert sum
is accumulated in fp32 and returned in the input's dtype. Dense SingleExpertWeights have no int4
form and are refused with a TypeError.
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
    # The dequant runs on the HIP kernel. Host tensors are staged to the current ROCm device
    # and the result is returned on their device, as the reference returns it on the input's.
    home = tensors.qweight.device
    dev = home if home.type == "cuda" else torch.device("cuda", torch.cuda.current_device())
    out = ops.dequantize(tensors.qweight.to(dev).contiguous(), tensors.qzeros.to(dev).contiguous(),
                         tensors.scales.to(device=dev, dtype=torch.float16).contiguous(),
                         tensors.g_idx.to(device=dev, dtype=torch.int32).contiguous(),
                         group_size=group_size, linear_weight=linear_weight, dtype=target_dtype)
    return out if home.type == "cuda" else out.to(home)


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
                                   device: str | torch.device = "cpu") -> torch.Tensor:
    tensors = load_repacked_projection_tensors(store, layer=layer, expert=expert,
                                               projection=projection, device=device)
    return dequantize_gptq_projection(tensors, bits=bits, dtype=dtype)


def apply_dequantized_projection(input_tensor: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    return F.linear(input_tensor, weight)


def load_single_expert_weights(store: RepackedMoeExpertStore, *, layer: int, expert: int,
                               bits: int = 4, dtype: str | torch.dtype = torch.bfloat16,
                               device: str | torch.device = "cpu") -> SingleExpertWeights:
    """Dense dequantised weights of one expert (HIP dequant kernel)."""
    projs = {p: dequantize_repacked_projection(store, layer=layer, expert=expert, projection=p,
                                               bits=bits, dtype=dtype, device=device)
             for p in ("gate_proj", "up_proj", "down_proj")}
    weights = SingleExpertWeights(projs["gate_proj"], projs["up_proj"], projs["down_proj"])
    _validate_single_expert_weights(weights)
    return weights


def _as_quantized(weights) -> QuantizedExpertWeights:
    if isinstance(weights, QuantizedExpertWeights):
        return weights
    if isinstance(weights, SingleExpertWeights):
        raise TypeError(
            "SingleExpertMlp runs int4 GPTQ experts on the W4A16 kernels and takes "
            "QuantizedExpertWeights (load_single_expert_mlp / load_quantized_expert); dense "
            "SingleExpertWeights have no int4 form to run")
    raise TypeError(f"expected QuantizedExpertWeights, got {type(weights).__name__}")


_KINDS = ("qweight", "qzeros", "scales")
_MAX_IDS_PER_CALL = 64  # experts per token that one fused-experts call accepts


class _Int4ExpertStack(torch.nn.Module):
    """int4 GPTQ stacks of n experts held as non-persistent buffers
    ``{proj}_{kind}`` ([n, ...]), so ``parameters()/buffers()``, ``.to()`` and ``.cuda()`` see
    and move them as they see the reference modules' dense weight buffers. The MoeExperts view
    the kernels take is rebuilt from the buffers after every move."""

    def _init_stack(self, experts: list[QuantizedExpertWeights], dtype) -> None:
        self.compute_dtype = resolve_torch_dtype(dtype)
        if self.compute_dtype not in ops.OUT_DTYPES:
            raise ValueError(f"Unsupported dtype {self.compute_dtype}")
        group = experts[0].group_size
        stacks = {}
        for proj in ("gate_proj", "up_proj", "down_proj"):
            ps = [getattr(e, proj) for e in experts]
            st = GptqStack(torch.stack([p.qweight for p in ps]).contiguous(),
                           torch.stack([p.qzeros for p in ps]).contiguous(),
                           torch.stack([p.scales.to(torch.float16) for p in ps]).contiguous(),
                           torch.stack([p.g_idx.to(torch.int32) for p in ps]).contiguous())
            stacks[proj] = st
        # shapes, dtypes and g_idx[k] == k // group are checked once, here
        MoeExperts(stacks["gate_proj"], stacks["up_proj"], stacks["down_proj"], group).validate()
        for proj, st in stacks.items():
            for kind in _KINDS:
                self.register_buffer(f"{proj}_{kind}", getattr(st, kind), persistent=False)
        self.group_size = int(group)
        self._view: MoeExperts | None = None
        self._dense: dict = {}
        self._staged: dict = {}

    def _apply(self, fn, recurse=True):
        out = super()._apply(fn, recurse)
        self._view = None
        self._dense = {}
        self._staged = {}
        return out

    def _stack_of(self, proj: str) -> GptqStack:
        return GptqStack(*(getattr(self, f"{proj}_{kind}") for kind in _KINDS))

    def int4_experts(self) -> MoeExperts:
        """The stacks as the kernels' MoeExperts (validated at construction)."""
        if self._view is None:
            view = MoeExperts(self._stack_of("gate_proj"), self._stack_of("up_proj"),
                              self._stack_of("down_proj"), self.group_size)
            view._validated = True
            self._view = view
        return self._view

    def _kernel_device(self, input_device: torch.device | None = None) -> torch.device:
        """Where the kernels run: the input's ROCm device, else the module's, else the current
        one (a host module and host inputs run there and return on the host, as the reference's
        CPU modules do; there is no CPU path)."""
        if input_device is not None and input_device.type == "cuda":
            return input_device
        home = self.gate_proj_qweight.device
        if home.type == "cuda":
            return home
        if not torch.cuda.is_available():
            raise RuntimeError("the W4A16 expert kernels run on a ROCm device and none is "
                               "available; there is no CPU fallback")
        return torch.device("cuda", torch.cuda.current_device())

    def _kernel_experts(self, dev: torch.device) -> MoeExperts:
        """The int4 stacks on ROCm device ``dev``: the module's buffers when they live there,
        else a copy staged once per device (dropped when the module moves)."""
        view = self.int4_experts()
        if view.device == dev:
            return view
        staged = self._staged.get(dev)
        if staged is None:
            staged = MoeExperts(view.gate.to(dev), view.up.to(dev), view.down.to(dev),
                                view.group_size)
            staged._validated = True
            self._staged[dev] = staged
        return staged

    def _dequantized(self, proj: str, row: int = 0) -> torch.Tensor:
        """Dense Linear-orientation weight of one projection of stack row ``row`` in the
        module's dtype, dequantised bit-exactly by the HIP kernel on first use and kept on the
        module's device."""
        key = (proj, row)
        if key not in self._dense:
            home = self.gate_proj_qweight.device
            dev = self._kernel_device()
            st = getattr(self._kernel_experts(dev), {"gate_proj": "gate", "up_proj": "up",
                                                      "down_proj": "down"}[proj])
            w = ops.dequantize(st.qweight[row], st.qzeros[row], st.scales[row],
                               group_size=self.group_size, linear_weight=True,
                               dtype=self.compute_dtype)
            self._dense[key] = w if home.type == "cuda" else w.to(home)
        return self._dense[key]

    @property
    def hidden_size(self) -> int:
        return int(self.gate_proj_qweight.shape[1]) * 8

    @property
    def intermediate_size(self) -> int:
        return int(self.gate_proj_qweight.shape[2])

    def _run(self, input_tensor: torch.Tensor, rows: list[int], weights: torch.Tensor | None):
        """out[t] = sum_i w_i * expert_{rows[i]}(x[t]) on the fused kernels. Activations enter
        the kernels as bf16 (fp16/fp32 inputs are rounded to bf16); the sum is accumulated in
        fp32 and returned in the input's dtype."""
        if input_tensor.shape[-1] != self.hidden_size:
            msg = f"Expected input last dim {self.hidden_size}, got {input_tensor.shape[-1]}"
            raise ValueError(msg)
        if input_tensor.dtype not in ops.OUT_DTYPES:
            raise TypeError(f"input dtype {input_tensor.dtype} is not one of bf16/fp16/fp32")
        # Host modules or host inputs (the reference's device="cpu" default) are staged to the
        # ROCm device the kernels run on; the result returns on the input's device.
        home = input_tensor.device
        dev = self._kernel_device(home)
        experts = self._kernel_experts(dev)
        x = input_tensor.reshape(-1, self.hidden_size).to(device=dev, dtype=torch.bfloat16)
        x = x.contiguous()
        T, k = x.shape[0], len(rows)
        if k == 0:  # the reference's sum over no experts is its zero start value
            return torch.zeros_like(input_tensor)
        ids = torch.tensor(rows, dtype=torch.int32, device=dev).expand(T, k).contiguous()
        if weights is None:
            w = torch.ones(T, k, dtype=torch.float32, device=dev)
        else:
            w = weights.to(device=dev, dtype=torch.float32).expand(T, k).contiguous()
        if k <= _MAX_IDS_PER_CALL:
            out = ops.fused_experts(x, ids, w, experts)
        else:  # the kernels take up to 64 experts per token: sum the chunks' outputs in fp32
            out = torch.zeros(T, self.hidden_size, dtype=torch.float32, device=dev)
            for lo in range(0, k, _MAX_IDS_PER_CALL):
                hi = min(lo + _MAX_IDS_PER_CALL, k)
                out += ops.fused_experts(x, ids[:, lo:hi].contiguous(), w[:, lo:hi].contiguous(),
                                         experts).float()
        return out.to(device=home, dtype=input_tensor.dtype).reshape(input_tensor.shape)


class SingleExpertMlp(_Int4ExpertStack):
    """y = W_down (silu(W_gate x) * (W_up x)) on int4 weights (gptq_unpack.py:231-256).

    ``gate_proj`` / ``up_proj`` / ``down_proj`` are the dense Linear-orientation weights the
    reference module holds, dequantised bit-exactly on first access in ``dtype``; the forward
    reads the int4 buffers, never the dense copies."""

    def __init__(self, weights: QuantizedExpertWeights, *,
                 dtype: str | torch.dtype = torch.bfloat16) -> None:
        super().__init__()
        q = _as_quantized(weights)
        self._init_stack([q], dtype)

    @property
    def gate_proj(self) -> torch.Tensor:
        return self._dequantized("gate_proj")

    @property
    def up_proj(self) -> torch.Tensor:
        return self._dequantized("up_proj")

    @property
    def down_proj(self) -> torch.Tensor:
        return self._dequantized("down_proj")

    def quantized(self) -> QuantizedExpertWeights:
        """The expert's int4 tensors (views of this module's buffers)."""
        projs = {}
        for proj in ("gate_proj", "up_proj", "down_proj"):
            st = self._stack_of(proj)
            g = torch.arange(st.in_features, dtype=torch.int32, device=st.qweight.device)
            projs[proj] = GptqProjectionTensors(st.qweight[0], st.qzeros[0], st.scales[0],
                                                g // self.group_size)
        return QuantizedExpertWeights(projs["gate_proj"], projs["up_proj"], projs["down_proj"],
                                      self.group_size)

    def forward(self, input_tensor: torch.Tensor) -> torch.Tensor:
        return self._run(input_tensor, [0], None)


class TopKExpertMlp(_Int4ExpertStack):
    """sum_i w_i * expert_{id_i}(x) over one shared expert set (gptq_unpack.py:259-327).

    The loaded experts are stacked in ascending id order into one int4 stack (buffers
    ``{proj}_{kind}`` [n, ...]); ``experts`` maps str(id) to a SingleExpertMlp over that
    expert's rows, as the reference's ModuleDict does."""

    def __init__(self, experts: dict[int, SingleExpertMlp | QuantizedExpertWeights], *,
                 dtype: str | torch.dtype | None = None) -> None:
        super().__init__()
        if not experts:
            msg = "TopKExpertMlp requires at least one expert"
            raise ValueError(msg)
        dtypes = {v.compute_dtype for v in experts.values() if isinstance(v, SingleExpertMlp)}
        quant = {int(k): (v.quantized() if isinstance(v, SingleExpertMlp) else _as_quantized(v))
                 for k, v in experts.items()}
        hidden_sizes = {q.hidden_size for q in quant.values()}
        intermediate_sizes = {q.intermediate_size for q in quant.values()}
        if len(hidden_sizes) != 1 or len(intermediate_sizes) != 1:
            msg = (f"All experts must share dimensions; got hidden={hidden_sizes}, "
                   f"intermediate={intermediate_sizes}")
            raise ValueError(msg)
        if dtype is None:
            dtype = dtypes.pop() if len(dtypes) == 1 else torch.bfloat16
        self._ids = tuple(sorted(quant))
        self._init_stack([quant[i] for i in self._ids], dtype)
        self._row = {eid: row for row, eid in enumerate(self._ids)}

    @property
    def loaded_expert_ids(self) -> tuple[int, ...]:
        return self._ids

    @property
    def experts(self) -> dict[str, SingleExpertMlp]:
        out = {}
        for eid, row in self._row.items():
            projs = {}
            for proj in ("gate_proj", "up_proj", "down_proj"):
                st = self._stack_of(proj)
                g = torch.arange(st.in_features, dtype=torch.int32, device=st.qweight.device)
                projs[proj] = GptqProjectionTensors(st.qweight[row], st.qzeros[row],
                                                    st.scales[row], g // self.group_size)
            out[str(eid)] = SingleExpertMlp(
                QuantizedExpertWeights(projs["gate_proj"], projs["up_proj"], projs["down_proj"],
                                       self.group_size), dtype=self.compute_dtype)
        return out

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
        # the reference casts the routing weights to the input's device and dtype (:319)
        w = expert_weights.to(device=input_tensor.device, dtype=input_tensor.dtype)
        return self._run(input_tensor, rows, w)


def load_quantized_expert(store: RepackedMoeExpertStore, *, layer: int, expert: int,
                          device: str | torch.device = "cpu") -> QuantizedExpertWeights:
    projs = {p: load_repacked_projection_tensors(store, layer=layer, expert=expert, projection=p,
                                                 device=device)
             for p in ("gate_proj", "up_proj", "down_proj")}
    group = int(projs["gate_proj"].qweight.shape[0]) * 8 // int(projs["gate_proj"].scales.shape[0])
    return QuantizedExpertWeights(projs["gate_proj"], projs["up_proj"], projs["down_proj"], group)


def _check_bits(bits: int) -> None:
    _validate_bits(bits)
    if bits != 4:
        raise NotImplementedError("the fused expert kernels implement 4-bit GPTQ")


def load_single_expert_mlp(store: RepackedMoeExpertStore, *, layer: int, expert: int,
                           bits: int = 4, dtype: str | torch.dtype = torch.bfloat16,
                           device: str | torch.device = "cpu") -> SingleExpertMlp:
    _check_bits(bits)
    return SingleExpertMlp(load_quantized_expert(store, layer=layer, expert=expert, device=device),
                           dtype=dtype)


def load_topk_expert_mlp(store: RepackedMoeExpertStore, *, layer: int,
                         expert_ids: list[int] | tuple[int, ...], bits: int = 4,
                         dtype: str | torch.dtype = torch.bfloat16,
                         device: str | torch.device = "cpu") -> TopKExpertMlp:
    _check_bits(bits)
    unique_expert_ids = tuple(dict.fromkeys(int(expert_id) for expert_id in expert_ids))
    experts = {eid: load_quantized_expert(store, layer=layer, expert=eid, device=device)
               for eid in unique_expert_ids}
    return TopKExpertMlp(experts, dtype=dtype)


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
