"""Qwen3-MoE GPTQ checkpoint -> repacked expert store, the format RepackedMoeExpertStore reads.

Reference: src/mtp_expert_prefetch/repack/qwen3_moe_gptq.py (key pattern :16-20, repack_layer
:142-198, repack_qwen3_moe_gptq :201-265, load_repack_manifest :268-284,
verify_random_repacked_slices :287-377). Same input (a Hugging Face safetensors snapshot: shards
plus model.safetensors.index.json), same output (per layer `layer_XX.safetensors` holding
`experts.{projection}.{kind}` stacked over experts [E, ...], `manifest.jsonl` with one JSON
record per layer, `summary.json`), the same record and summary fields, layer selection syntax
("0,2,5-7") and errors, so a store written by either tool reads the same.

Host-side file work (safetensors reads and writes); nothing here runs on the GPU.
"""

from __future__ import annotations

import json
import random
import re
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from mtp_amd.repack.store import KINDS, PROJECTIONS, tensor_sha256

# model.language_model.layers.<L>.mlp.experts.<E>.<projection>.<kind>
EXPERT_KEY_RE = re.compile(
    r"^(?P<prefix>model\.language_model\.layers\.(?P<layer>\d+)\.mlp\.experts)"
    r"\.(?P<expert>\d+)\.(?P<projection>down_proj|gate_proj|up_proj)"
    r"\.(?P<kind>g_idx|qweight|qzeros|scales)$")


@dataclass(frozen=True)
class ExpertKey:
    key: str
    layer: int
    expert: int
    projection: str
    kind: str


def _dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).replace("torch.", "")


def _source_key(layer: int, expert: int | str, projection: str, kind: str) -> str:
    return f"model.language_model.layers.{layer}.mlp.experts.{expert}.{projection}.{kind}"


class ShardedSafeTensorReader:
    """Tensors of a sharded snapshot by key, through the index's weight map (one open handle per
    shard, kept for the reader's lifetime)."""

    def __init__(self, snapshot_path: Path) -> None:
        self.snapshot_path = Path(snapshot_path)
        self.index_path = self.snapshot_path / "model.safetensors.index.json"
        if not self.index_path.exists():
            raise FileNotFoundError(f"Missing safetensors index: {self.index_path}")
        self.index = json.loads(self.index_path.read_text(encoding="utf-8"))
        self.weight_map: dict[str, str] = self.index["weight_map"]
        self._handles: dict[str, Any] = {}

    def get_tensor(self, key: str) -> torch.Tensor:
        shard = self.weight_map[key]
        if shard not in self._handles:
            path = self.snapshot_path / shard
            if not path.exists():
                raise FileNotFoundError(f"Missing shard for {key}: {path}")
            self._handles[shard] = safe_open(str(path), framework="pt", device="cpu")
        return self._handles[shard].get_tensor(key)


def parse_expert_key(key: str) -> ExpertKey | None:
    m = EXPERT_KEY_RE.match(key)
    if m is None:
        return None
    return ExpertKey(key, int(m["layer"]), int(m["expert"]), m["projection"], m["kind"])


def discover_expert_keys(weight_map: dict[str, str]) -> dict[int, dict[str, dict[str, dict[int, str]]]]:
    """layer -> projection -> kind -> expert -> source key, for every expert tensor of the map."""
    out: dict[int, dict[str, dict[str, dict[int, str]]]] = {}
    for key in weight_map:
        k = parse_expert_key(key)
        if k is not None:
            out.setdefault(k.layer, {}).setdefault(k.projection, {}).setdefault(k.kind, {})[
                k.expert] = key
    return out


def parse_layers(layers: str | None, available_layers: list[int]) -> list[int]:
    """Layers named by "a,b,c-d" (None: all), in checkpoint order; unknown layers raise."""
    if layers is None:
        return list(available_layers)
    wanted: set[int] = set()
    for token in (t.strip() for t in layers.split(",")):
        if not token:
            continue
        if "-" in token:
            lo, hi = (int(v) for v in token.split("-", 1))
            if hi < lo:
                raise ValueError(f"Invalid descending layer range: {token}")
            wanted.update(range(lo, hi + 1))
        else:
            wanted.add(int(token))
    unknown = sorted(wanted - set(available_layers))
    if unknown:
        raise ValueError(f"Requested layers are not present in checkpoint: {unknown}")
    return [layer for layer in available_layers if layer in wanted]


def _layer_source_keys(group: dict[str, dict[str, dict[int, str]]], layer: int, projection: str,
                       kind: str, num_experts: int) -> list[str]:
    by_expert = group.get(projection, {}).get(kind, {})
    missing = [e for e in range(num_experts) if e not in by_expert]
    if missing:
        more = "..." if len(missing) > 16 else ""
        raise RuntimeError(f"Layer {layer} {projection}.{kind} is missing {len(missing)} experts: "
                           f"{missing[:16]}{more}")
    return [by_expert[e] for e in range(num_experts)]


def repack_layer(reader: ShardedSafeTensorReader,
                 grouped_keys: dict[int, dict[str, dict[str, dict[int, str]]]], *, layer: int,
                 output_dir: Path, num_experts: int, verify: bool) -> dict[str, Any]:
    """Stack the layer's 12 per-expert tensor families into layer_XX.safetensors; returns the
    layer's manifest record."""
    group = grouped_keys[layer]
    stacked_out: dict[str, torch.Tensor] = {}
    records: dict[str, Any] = {}
    for projection in PROJECTIONS:
        for kind in KINDS:
            keys = _layer_source_keys(group, layer, projection, kind, num_experts)
            pieces = [reader.get_tensor(k) for k in keys]
            stacked = torch.stack(pieces, dim=0).contiguous()
            name = f"experts.{projection}.{kind}"
            if verify:
                for e, piece in enumerate(pieces):
                    if not torch.equal(stacked[e], piece):
                        raise RuntimeError(f"Repack verification failed for layer={layer} {name} "
                                           f"expert={e}")
            stacked_out[name] = stacked
            records[name] = {
                "shape": list(stacked.shape),
                "dtype": _dtype_name(stacked.dtype),
                "sha256": tensor_sha256(stacked),
                "source_count": len(keys),
                "source_shape": list(pieces[0].shape),
                "source_dtype": _dtype_name(pieces[0].dtype),
                "source_key_template": _source_key(layer, "{expert}", projection, kind),
            }
    path = Path(output_dir) / f"layer_{layer:02d}.safetensors"
    save_file(stacked_out, str(path))
    return {"layer": layer, "path": path.name, "num_experts": num_experts,
            "num_source_tensors": len(PROJECTIONS) * len(KINDS) * num_experts,
            "num_output_tensors": len(stacked_out), "tensors": records}


def repack_qwen3_moe_gptq(snapshot_path: Path, output_dir: Path, *, layers: str | None = None,
                          num_experts: int = 256, verify: bool = False,
                          overwrite: bool = False) -> Path:
    """Repack the selected layers of a snapshot into output_dir; returns manifest.jsonl's path.
    An existing manifest is kept unless overwrite is set."""
    snapshot_path = Path(snapshot_path).expanduser().resolve()
    output_dir = Path(output_dir).expanduser().resolve()
    output_dir.mkdir(parents=True, exist_ok=True)
    manifest_path = output_dir / "manifest.jsonl"
    if manifest_path.exists() and not overwrite:
        raise FileExistsError(f"Refusing to overwrite existing manifest: {manifest_path}. "
                              "Pass --overwrite.")
    reader = ShardedSafeTensorReader(snapshot_path)
    grouped = discover_expert_keys(reader.weight_map)
    selected = parse_layers(layers, sorted(grouped))
    if not selected:
        raise RuntimeError("No expert layers selected for repacking.")
    n_src = n_out = 0
    with manifest_path.open("w", encoding="utf-8") as manifest:
        for layer in selected:
            rec = repack_layer(reader, grouped, layer=layer, output_dir=output_dir,
                               num_experts=num_experts, verify=verify)
            n_src += int(rec["num_source_tensors"])
            n_out += int(rec["num_output_tensors"])
            manifest.write(json.dumps(rec, sort_keys=True) + "\n")
            print(f"repacked layer {layer:02d}: {rec['num_source_tensors']} -> "
                  f"{rec['num_output_tensors']} tensors")
    summary = {
        "snapshot_path": str(snapshot_path), "output_dir": str(output_dir),
        "manifest_path": manifest_path.name, "layers": selected, "num_layers": len(selected),
        "num_experts": num_experts, "projections": list(PROJECTIONS), "kinds": list(KINDS),
        "total_source_tensors": n_src, "total_output_tensors": n_out,
        "reduction_factor": n_src / n_out if n_out else None, "verify": verify,
    }
    (output_dir / "summary.json").write_text(json.dumps(summary, indent=2, sort_keys=True) + "\n",
                                             encoding="utf-8")
    return manifest_path


def load_repack_manifest(repacked_dir: Path) -> dict[int, dict[str, Any]]:
    """layer -> manifest record of a repacked store."""
    path = Path(repacked_dir) / "manifest.jsonl"
    if not path.exists():
        raise FileNotFoundError(f"Missing repack manifest: {path}")
    records: dict[int, dict[str, Any]] = {}
    for line in path.read_text(encoding="utf-8").splitlines():
        if line.strip():
            rec = json.loads(line)
            records[int(rec["layer"])] = rec
    if not records:
        raise RuntimeError(f"Repack manifest is empty: {path}")
    return records


def verify_random_repacked_slices(snapshot_path: Path, repacked_dir: Path, *, samples: int = 128,
                                  seed: int = 0, layers: str | None = None,
                                  num_experts: int | None = None,
                                  fail_fast: bool = True) -> dict[str, Any]:
    """Compare `samples` random (layer, expert, projection, kind) slices of the store with the
    snapshot's source tensors (random.Random(seed) draws layer, expert, projection, kind in
    that order, as the reference does, so a seed checks the same slices)."""
    snapshot_path = Path(snapshot_path).expanduser().resolve()
    repacked_dir = Path(repacked_dir).expanduser().resolve()
    reader = ShardedSafeTensorReader(snapshot_path)
    manifest = load_repack_manifest(repacked_dir)
    selected = parse_layers(layers, sorted(manifest))
    if not selected:
        raise RuntimeError("No repacked layers selected for verification.")
    if num_experts is None:
        num_experts = int(next(iter(manifest.values())).get("num_experts", 256))
    rng = random.Random(seed)
    handles: dict[int, Any] = {}
    checked: list[dict[str, Any]] = []
    failures: list[dict[str, Any]] = []
    for i in range(samples):
        layer = rng.choice(selected)
        expert = rng.randrange(num_experts)
        projection = rng.choice(PROJECTIONS)
        kind = rng.choice(KINDS)
        src_key = _source_key(layer, expert, projection, kind)
        rep_key = f"experts.{projection}.{kind}"
        if layer not in handles:
            path = repacked_dir / manifest[layer]["path"]
            if not path.exists():
                raise FileNotFoundError(f"Missing repacked layer file: {path}")
            handles[layer] = safe_open(str(path), framework="pt", device="cpu")
        original = reader.get_tensor(src_key)
        fused = handles[layer].get_tensor(rep_key)
        if expert >= fused.shape[0]:
            raise RuntimeError(f"Expert index {expert} is out of range for {rep_key}: "
                               f"{list(fused.shape)}")
        restored = fused[expert]
        ok = torch.equal(original, restored)
        rec = {"sample_idx": i, "layer": layer, "expert": expert, "projection": projection,
               "kind": kind, "source_key": src_key, "repacked_key": rep_key,
               "source_shape": list(original.shape), "repacked_slice_shape": list(restored.shape),
               "dtype": _dtype_name(original.dtype), "ok": ok}
        checked.append(rec)
        if not ok:
            rec["source_sha256"] = tensor_sha256(original)
            rec["repacked_slice_sha256"] = tensor_sha256(restored)
            failures.append(rec)
            if fail_fast:
                break
    return {"snapshot_path": str(snapshot_path), "repacked_dir": str(repacked_dir),
            "samples_requested": samples, "samples_checked": len(checked), "seed": seed,
            "layers": selected, "num_experts": num_experts, "failures": failures,
            "ok": not failures}
