"""HiddenResidualExpertPredictor on the HIP kernels (moe_hr_predictor_v1).

Mirrors the reference's module (src/mtp_expert_prefetch/training/hidden_residual.py:44-121):
the same constructor arguments, forward(hidden, *, layer_ids) -> residual logits
[examples, future_window, num_experts], apply_residual_scale with a fixed or learnt (softplus)
gamma, and the same error messages; load_reference_state_dict takes the reference's parameter
names (encoder.0.*, encoder.2.*, layer_embedding, delta_embedding, classifier, raw_residual_gamma).
Inference only: parameters are bf16 (biases kept as fp32 copies of bf16 values), activations
between the Linear layers are bf16, and the dot products use the router's canonical fp32 order.
predict_topk adds the residual to prior logits (prior + gamma * residual, the training script's
combination, train_hidden_residual_predictor_smoke.py:446) and returns the top-k experts of every
(example, future delta) for the slot cache's prefetch.
"""

from __future__ import annotations

import ctypes
import math

import torch
import torch.nn.functional as F

from mtp_amd import _lib


def _inverse_softplus(value: float) -> float:
    if value > 20.0:
        return value
    return math.log(math.expm1(value))


class HiddenResidualExpertPredictor(torch.nn.Module):
    def __init__(self, *, hidden_size: int = 2048, num_experts: int = 256, num_layers: int = 40,
                 future_window: int = 4, width: int = 256, dropout: float = 0.0,
                 zero_init_output: bool = False, learnable_residual_gamma: bool = False,
                 initial_residual_gamma: float = 1.0, residual_gamma_scope: str = "scalar",
                 ln_eps: float = 1e-5, seed: int = 0, device: str | torch.device = "cuda") -> None:
        super().__init__()
        self.hidden_size = int(hidden_size)
        self.num_experts = int(num_experts)
        self.num_layers = int(num_layers)
        self.future_window = int(future_window)
        self.width = int(width)
        self.dropout = float(dropout)  # inference: dropout is the identity
        self.ln_eps = float(ln_eps)
        self.learnable_residual_gamma = bool(learnable_residual_gamma)
        self.residual_gamma_scope = str(residual_gamma_scope)
        g = torch.Generator().manual_seed(int(seed))
        # torch.nn.Linear / Embedding / LayerNorm default initialisation, then bf16
        bound_enc = 1.0 / math.sqrt(self.hidden_size)
        bound_cls = 1.0 / math.sqrt(self.width)

        def uni(shape, b):
            return (torch.rand(shape, generator=g) * 2 - 1) * b
        params = {
            "enc_w": uni((self.width, self.hidden_size), bound_enc),
            "enc_b": uni((self.width,), bound_enc),
            "ln_w": torch.ones(self.width),
            "ln_b": torch.zeros(self.width),
            "layer_emb": torch.randn((self.num_layers, self.width), generator=g),
            "delta_emb": torch.randn((self.future_window, self.width), generator=g),
            "cls_w": uni((self.num_experts, self.width), bound_cls),
            "cls_b": uni((self.num_experts,), bound_cls),
        }
        if zero_init_output:
            params["cls_w"].zero_()
            params["cls_b"].zero_()
        for name, t in params.items():
            self._set(name, t, device)
        if self.learnable_residual_gamma:
            if self.residual_gamma_scope not in {"scalar", "layer"}:
                msg = "residual_gamma_scope must be 'scalar' or 'layer'."
                raise ValueError(msg)
            gamma = max(float(initial_residual_gamma), 1e-8)
            shape = (self.num_layers,) if self.residual_gamma_scope == "layer" else ()
            self.raw_residual_gamma = torch.nn.Parameter(
                torch.full(shape, _inverse_softplus(gamma), device=device), requires_grad=False)
        else:
            self.register_parameter("raw_residual_gamma", None)
        self._ws: torch.Tensor | None = None

    def _set(self, name: str, t: torch.Tensor, device) -> None:
        if name in ("enc_b", "cls_b"):  # fp32 holding bf16 values
            t = t.to(torch.bfloat16).to(torch.float32)
        else:
            t = t.to(torch.bfloat16)
        self.register_buffer(name, t.contiguous().to(device), persistent=True)

    def load_reference_state_dict(self, state: dict[str, torch.Tensor]) -> None:
        """Parameters of a trained reference module (its state_dict names)."""
        names = {"encoder.0.weight": "enc_w", "encoder.0.bias": "enc_b", "encoder.2.weight": "ln_w",
                 "encoder.2.bias": "ln_b", "layer_embedding.weight": "layer_emb",
                 "delta_embedding.weight": "delta_emb", "classifier.weight": "cls_w",
                 "classifier.bias": "cls_b"}
        for key, name in names.items():
            if key not in state:
                raise KeyError(f"missing {key} in the predictor state dict")
            src = state[key]
            if tuple(src.shape) != tuple(getattr(self, name).shape):
                raise ValueError(f"{key}: shape {tuple(src.shape)} != {tuple(getattr(self, name).shape)}")
            self._set(name, src.detach().float(), getattr(self, name).device)
        if "raw_residual_gamma" in state and self.raw_residual_gamma is not None:
            self.raw_residual_gamma.data.copy_(state["raw_residual_gamma"].to(self.raw_residual_gamma))

    def _params(self) -> _lib.HrPredictorParams:
        return _lib.HrPredictorParams(
            self.enc_w.data_ptr(), self.enc_b.data_ptr(), self.ln_w.data_ptr(), self.ln_b.data_ptr(),
            self.layer_emb.data_ptr(), self.delta_emb.data_ptr(), self.cls_w.data_ptr(),
            self.cls_b.data_ptr(), self.hidden_size, self.width, self.num_layers,
            self.future_window, self.num_experts, self.ln_eps)

    def _check(self, hidden: torch.Tensor, layer_ids: torch.Tensor) -> None:
        if hidden.ndim != 2 or hidden.shape[-1] != self.hidden_size:
            msg = f"Expected hidden [examples, {self.hidden_size}], got {tuple(hidden.shape)}"
            raise ValueError(msg)
        if layer_ids.ndim != 1 or layer_ids.shape[0] != hidden.shape[0]:
            msg = ("layer_ids must have shape [examples] matching hidden, "
                   f"got {tuple(layer_ids.shape)} and {tuple(hidden.shape)}")
            raise ValueError(msg)

    def _run(self, hidden, layer_ids, top_k, prior=None, scale=1.0, scale_per_example=None):
        lib = _lib.load()
        self._check(hidden, layer_ids)
        dev = self.enc_w.device
        if dev.type != "cuda":
            raise ValueError("the predictor kernels run on a ROCm device (move it with .to('cuda'))")
        x = hidden.to(device=dev, dtype=torch.bfloat16).contiguous()
        ids_l = layer_ids.to(device=dev, dtype=torch.int32).contiguous()
        N = x.shape[0]
        p = self._params()
        need = int(lib.moe_hr_predictor_workspace_bytes_v1(N, ctypes.byref(p)))
        if self._ws is None or self._ws.numel() < need or self._ws.device != dev:
            self._ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        out = torch.empty(N, self.future_window, self.num_experts, dtype=torch.float32, device=dev)
        ids = torch.empty(N, self.future_window, top_k, dtype=torch.int32, device=dev)
        pr = None
        if prior is not None:
            pr = prior.to(device=dev, dtype=torch.float32).expand(
                N, self.future_window, self.num_experts).contiguous()
        spe = None if scale_per_example is None else scale_per_example.to(
            device=dev, dtype=torch.float32).contiguous()
        _lib.check(lib.moe_hr_predictor_v1(
            x.data_ptr(), N, ids_l.data_ptr(), ctypes.byref(p), None if pr is None else pr.data_ptr(),
            float(scale), None if spe is None else spe.data_ptr(), int(top_k), self._ws.data_ptr(),
            self._ws.numel(), out.data_ptr(), ids.data_ptr(),
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
        return out, ids

    def forward(self, hidden: torch.Tensor, *, layer_ids: torch.Tensor) -> torch.Tensor:
        out, _ = self._run(hidden, layer_ids, 1)
        return out

    def _gamma(self, layer_ids: torch.Tensor, fixed_scale: float):
        """(scalar scale, per-example scales or None) of apply_residual_scale (:108-121)."""
        if self.raw_residual_gamma is None:
            return float(fixed_scale), None
        gamma = F.softplus(self.raw_residual_gamma.float())
        if self.residual_gamma_scope == "layer":
            return 1.0, gamma[layer_ids.to(device=gamma.device, dtype=torch.long)]
        return float(gamma), None

    def apply_residual_scale(self, residual: torch.Tensor, *, layer_ids: torch.Tensor,
                             fixed_scale: float) -> torch.Tensor:
        scale, per = self._gamma(layer_ids, fixed_scale)
        if per is None:
            return scale * residual
        return per[:, None, None].to(dtype=residual.dtype) * residual

    def predict_topk(self, hidden: torch.Tensor, *, layer_ids: torch.Tensor, k: int,
                     prior: torch.Tensor | None = None, fixed_scale: float = 1.0,
                     return_logits: bool = False):
        """Top-k experts of prior + gamma * residual for every (example, future delta):
        int32 [examples, future_window, k] (and the combined fp32 logits)."""
        scale, per = self._gamma(layer_ids, fixed_scale)
        out, ids = self._run(hidden, layer_ids, k, prior=prior, scale=scale, scale_per_example=per)
        return (ids, out) if return_logits else ids
