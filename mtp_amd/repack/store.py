"""Reader of the reference's repacked expert store (the L0 on-disk format).

Format (src/mtp_expert_prefetch/repack/qwen3_moe_gptq.py:142-198 and store.py:39-245):
  <dir>/summary.json          {"num_experts", "projections", "kinds", ...}
  <dir>/manifest.jsonl        one record per layer: {"layer", "path", "num_experts",
                              "tensors": {key: {"shape", "dtype", "sha256"}}}
  <dir>/layer_XX.safetensors  keys "experts.{proj}.{kind}" stacked over experts.
Same public names and errors as the reference's RepackedMoeExpertStore, plus
``load_layer`` which returns a whole layer as a device-resident MoeExperts. Stores are written
from a checkpoint snapshot by mtp_amd.repack.qwen3_moe_gptq.repack_qwen3_moe_gptq.
"""

from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import torch
from safetensors import safe_open

PROJECTIONS = ("down_proj", "gate_proj", "up_proj")
KINDS = ("g_idx", "qweight", "qzeros", "scales")
SAFETENSORS_DTYPE_NAMES = {"BOOL": "bool", "F16": "float16", "BF16": "bfloat16", "F32": "float32",
                           "F64": "float64", "I8": "int8", "I16": "int16", "I32": "int32",
                           "I64": "int64", "U8": "uint8"}


def tensor_sha256(tensor: torch.Tensor) -> str:
    """sha256 of the tensor's contiguous CPU bytes (bf16 hashed through its int16 view)."""
    t = tensor.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()


def normalize_safetensors_dtype(dtype: str) -> str:
    return SAFETENSORS_DTYPE_NAMES.get(dtype, dtype)


@dataclass(frozen=True)
class RepackedTensorInfo:
    layer: int
    projection: str
    kind: str
    key: str
    shape: tuple[int, ...]
    dtype: str
    sha256: str | None = None


class RepackedMoeExpertStore:
    """Lazy accessor for per-layer repacked Qwen3 MoE expert tensors."""

    def __init__(self, repacked_dir: str | Path, *, device: str = "cpu") -> None:
        self.repacked_dir = Path(repacked_dir).expanduser().resolve()
        self.device = device
        self.summary = self._read_summary()
        self.manifest = self._read_manifest()
        self.layers = tuple(sorted(self.manifest))
        if not self.layers:
            raise RuntimeError(f"No layers found in repack manifest: {self.repacked_dir}")
        first = self.manifest[self.layers[0]]
        self.num_experts = int(self.summary.get("num_experts", first["num_experts"]))
        self.projections = tuple(self.summary.get("projections", PROJECTIONS))
        self.kinds = tuple(self.summary.get("kinds", KINDS))
        self._handles: dict[int, Any] = {}

    def _read_summary(self) -> dict[str, Any]:
        path = self.repacked_dir / "summary.json"
        if not path.exists():
            raise FileNotFoundError(f"Missing repack summary: {path}")
        data = json.loads(path.read_text(encoding="utf-8"))
        if not isinstance(data, dict):
            raise TypeError(f"Expected mapping in repack summary: {path}")
        return data

    def _read_manifest(self) -> dict[int, dict[str, Any]]:
        path = self.repacked_dir / "manifest.jsonl"
        if not path.exists():
            raise FileNotFoundError(f"Missing repack manifest: {path}")
        records: dict[int, dict[str, Any]] = {}
        for line_no, line in enumerate(path.read_text(encoding="utf-8").splitlines(), start=1):
            if not line.strip():
                continue
            rec = json.loads(line)
            layer = int(rec["layer"])
            if layer in records:
                raise RuntimeError(f"Duplicate layer {layer} in {path}:{line_no}")
            records[layer] = rec
        return records

    def close(self) -> None:
        self._handles.clear()

    def __enter__(self) -> "RepackedMoeExpertStore":
        return self

    def __exit__(self, *_exc: object) -> None:
        self.close()

    def _record(self, layer: int) -> dict[str, Any]:
        try:
            return self.manifest[layer]
        except KeyError as exc:
            raise KeyError(f"Layer {layer} is not present in repacked store") from exc

    def layer_path(self, layer: int) -> Path:
        return self.repacked_dir / self._record(layer)["path"]

    def _check(self, projection: str, kind: str) -> None:
        if projection not in self.projections:
            raise ValueError(f"Unknown projection {projection!r}; expected one of {self.projections}")
        if kind not in self.kinds:
            raise ValueError(f"Unknown tensor kind {kind!r}; expected one of {self.kinds}")

    def tensor_key(self, projection: str, kind: str) -> str:
        self._check(projection, kind)
        return f"experts.{projection}.{kind}"

    def tensor_info(self, layer: int, projection: str, kind: str) -> RepackedTensorInfo:
        rec = self._record(layer)
        key = self.tensor_key(projection, kind)
        meta = rec.get("tensors", {}).get(key)
        if meta is None:
            raise KeyError(f"Missing tensor metadata for layer={layer} key={key}")
        return RepackedTensorInfo(layer, projection, kind, key, tuple(int(d) for d in meta["shape"]),
                                  str(meta["dtype"]), meta.get("sha256"))

    def _handle(self, layer: int):
        self._record(layer)
        h = self._handles.get(layer)
        if h is None:
            path = self.layer_path(layer)
            if not path.exists():
                raise FileNotFoundError(f"Missing repacked layer file: {path}")
            h = safe_open(path, framework="pt", device=self.device)
            self._handles[layer] = h
        return h

    def get_fused_tensor(self, layer: int, projection: str, kind: str) -> torch.Tensor:
        return self._handle(layer).get_tensor(self.tensor_key(projection, kind))

    def get_expert_tensor(self, layer: int, expert: int, projection: str, kind: str) -> torch.Tensor:
        if expert < 0 or expert >= self.num_experts:
            raise IndexError(f"Expert index out of range: expert={expert}, num_experts={self.num_experts}")
        return self._handle(layer).get_slice(self.tensor_key(projection, kind))[expert]

    def inspect(self, *, check_hashes: bool = False) -> dict[str, Any]:
        problems: dict[str, list] = {k: [] for k in ("missing_files", "missing_keys", "shape_mismatches",
                                                      "dtype_mismatches", "hash_mismatches")}
        for layer in self.layers:
            path = self.layer_path(layer)
            if not path.exists():
                problems["missing_files"].append(str(path))
                continue
            h = self._handle(layer)
            keys = set(h.keys())
            for proj in self.projections:
                for kind in self.kinds:
                    info = self.tensor_info(layer, proj, kind)
                    if info.key not in keys:
                        problems["missing_keys"].append({"layer": layer, "key": info.key})
                        continue
                    sl = h.get_slice(info.key)
                    shape = tuple(int(d) for d in sl.get_shape())
                    dtype = normalize_safetensors_dtype(str(sl.get_dtype()))
                    if shape != info.shape:
                        problems["shape_mismatches"].append(
                            {"layer": layer, "key": info.key, "expected": list(info.shape), "actual": list(shape)})
                    if dtype != info.dtype:
                        problems["dtype_mismatches"].append(
                            {"layer": layer, "key": info.key, "expected": info.dtype, "actual": dtype})
                    if check_hashes and info.sha256 is not None:
                        digest = tensor_sha256(h.get_tensor(info.key))
                        if digest != info.sha256:
                            problems["hash_mismatches"].append(
                                {"layer": layer, "key": info.key, "expected": info.sha256, "actual": digest})
        return {
            "ok": not any(problems.values()),
            "repacked_dir": str(self.repacked_dir),
            "layers": list(self.layers),
            "num_layers": len(self.layers),
            "num_experts": self.num_experts,
            "projections": list(self.projections),
            "kinds": list(self.kinds),
            "total_output_tensors": sum(int(r.get("num_output_tensors", 0)) for r in self.manifest.values()),
            **problems,
            "checked_hashes": check_hashes,
        }

    def read_layer_tensors(self, layer: int, *, verify: bool = True,
                           projections: tuple[str, ...] = ("gate_proj", "up_proj", "down_proj"),
                           kinds: tuple[str, ...] = ("qweight", "qzeros", "scales", "g_idx")
                           ) -> dict[str, torch.Tensor]:
        """The layer's stacked tensors {"experts.{proj}.{kind}": CPU tensor}, each checked
        against its manifest record (shape, dtype and, with verify, the sha256 that
        repack_layer wrote: qwen3_moe_gptq.py:112-118, 175-186). Raises ValueError on a
        mismatch, naming the layer and key."""
        out = {}
        for proj in projections:
            for kind in kinds:
                info = self.tensor_info(layer, proj, kind)
                t = self.get_fused_tensor(layer, proj, kind)
                shape = tuple(int(d) for d in t.shape)
                dtype = str(t.dtype).replace("torch.", "")
                if shape != info.shape:
                    raise ValueError(f"layer {layer} {info.key}: shape {list(shape)} != manifest "
                                     f"{list(info.shape)}")
                if dtype != info.dtype:
                    raise ValueError(f"layer {layer} {info.key}: dtype {dtype} != manifest {info.dtype}")
                if verify and info.sha256 is not None:
                    digest = tensor_sha256(t)
                    if digest != info.sha256:
                        raise ValueError(f"layer {layer} {info.key}: sha256 {digest} != manifest "
                                         f"{info.sha256}")
                out[info.key] = t
        return out

    def load_layer(self, layer: int, *, device: str | torch.device = "cuda", group_size: int | None = None,
                   verify: bool = True):
        """All experts of one layer as a device-resident MoeExperts (int4, repacked layout),
        verified against the manifest (read_layer_tensors) and copied host -> device through
        pinned staging. g_idx must be k // group_size (checked by MoeExperts.validate); the
        group size defaults to the one the tensors imply (in_features / scales rows)."""
        from mtp_amd.weights import GptqStack, MoeExperts

        t = self.read_layer_tensors(layer, verify=verify)
        dev = torch.device(device)
        stacks = {}
        for proj in ("gate_proj", "up_proj", "down_proj"):
            moved = []
            for kind in ("qweight", "qzeros", "scales", "g_idx"):
                src = t[f"experts.{proj}.{kind}"]
                if kind == "scales":
                    src = src.to(torch.float16)
                elif kind == "g_idx":
                    src = src.to(torch.int32)
                src = src.contiguous()
                if dev.type == "cuda":
                    src = src.pin_memory().to(dev, non_blocking=True)
                moved.append(src)
            stacks[proj] = GptqStack(*moved)
        if group_size is None:
            g = stacks["gate_proj"]
            group_size = g.in_features // int(g.scales.shape[1])
        experts = MoeExperts(stacks["gate_proj"], stacks["up_proj"], stacks["down_proj"], group_size)
        experts.validate()
        return experts


def write_repacked_store(out_dir: str | Path, layers: dict[int, dict[str, torch.Tensor]],
                         *, num_experts: int) -> Path:
    """Write already stacked layers ({key: stacked tensor}) in the repacked format (fixtures and
    tests; a checkpoint snapshot goes through qwen3_moe_gptq.repack_qwen3_moe_gptq)."""
    from safetensors.torch import save_file

    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    lines = []
    for layer, tensors in sorted(layers.items()):
        name = f"layer_{layer:02d}.safetensors"
        save_file({k: v.contiguous() for k, v in tensors.items()}, str(out / name))
        meta = {k: {"shape": list(v.shape), "dtype": str(v.dtype).replace("torch.", ""),
                    "sha256": tensor_sha256(v)} for k, v in tensors.items()}
        lines.append(json.dumps({"layer": layer, "path": name, "num_experts": num_experts,
                                 "num_output_tensors": len(tensors), "tensors": meta}))
    (out / "manifest.jsonl").write_text("\n".join(lines) + "\n", encoding="utf-8")
    (out / "summary.json").write_text(json.dumps({"num_experts": num_experts,
                                                  "projections": list(PROJECTIONS),
                                                  "kinds": list(KINDS)}), encoding="utf-8")
    return out
