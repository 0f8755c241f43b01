"""RoLaQ artifact loading and read-rotation folding (host side).

An artifact is a directory with ``manifest.json`` and one FP32 rotation per
decoder layer (``layer_<i>.pt``), in the format the reference writes
(mla_quant/quantizer.py:155-215). The drop-in entry points keep the
reference's names, arguments and ``ValueError`` behaviour:

* ``load_layer_quantizers(path, rotation_path, group_size, width, layer_ids)``
  -> per-layer ``(threshold, gain)`` or ``None`` without an artifact
  (deployment/sglang/srt/mem_cache/rolaq_mla.py:41-53);
* ``fold_read_rotation(weight, layer_id, rotation_path)`` -> ``bf16(W_b @
  fp32(bf16(R)))`` (rolaq_mla.py:56-71).

``Artifact`` gathers the checks the reference spreads over its loaders
(rolaq_mla.py:16-38, quantizer.py:145-152 and 217-252, deployment/serve.py:20-56):
manifest schema, every layer present, SHA-256 of every rotation file, finite
positive quantizer parameters, and -- when a rotation is read -- square, FP32,
finite and orthogonal to 1e-5. Rotations are read with
``torch.load(..., weights_only=True)`` only.
"""

from __future__ import annotations

import hashlib
import json
import math
from dataclasses import dataclass
from functools import lru_cache
from pathlib import Path

import torch

RECIPE = "learned_shared_latent_rotation_quantizer_v2"
FORMAT_VERSION = 2
GROUP_SIZE = 128

# manifest field -> the value a packed-INT2 (oscar_lloyd, content-only) artifact must hold
_REQUIRED = (
    ("recipe", RECIPE, "not a frozen v2 learned RoLaQ artifact"),
    ("family", "oscar_lloyd", "only the oscar_lloyd quantizer family is supported by the packed writer"),
    ("components", ["nope"], "expected a content-only (nope) artifact"),
    ("group_size", GROUP_SIZE, "expected quantization groups of 128"),
)


def file_sha256(path: Path) -> str:
    digest = hashlib.sha256()
    with Path(path).open("rb") as f:
        for block in iter(lambda: f.read(1 << 20), b""):
            digest.update(block)
    return digest.hexdigest()


def check_rotation(rotation, width: int | None, layer) -> torch.Tensor:
    """Square FP32, finite, ``|R^T R - I|_max <= 1e-5`` (quantizer.py:145-152)."""
    if not isinstance(rotation, torch.Tensor) or rotation.dtype != torch.float32 or rotation.dim() != 2 \
            or rotation.shape[0] != rotation.shape[1] or (width is not None and rotation.shape[0] != width):
        raise ValueError(f"layer {layer}: rotation must be a square FP32 matrix of the latent width")
    if not bool(torch.isfinite(rotation).all()):
        raise ValueError(f"layer {layer}: rotation has non-finite entries")
    r = rotation.double()
    residual = float((r.T @ r - torch.eye(r.shape[0], dtype=torch.float64)).abs().max())
    if residual > 1e-05:
        raise ValueError(f"layer {layer}: rotation is not orthogonal (residual {residual:.3g})")
    return rotation


@dataclass(frozen=True)
class LayerRecord:
    file: str
    sha256: str
    threshold: float
    gain: float


class Artifact:
    """A validated artifact directory (manifest checked on construction)."""

    def __init__(self, path):
        self.root = Path(path).resolve()
        manifest = json.loads((self.root / "manifest.json").read_text())
        for key, want, why in _REQUIRED:
            if manifest.get(key) != want:
                raise ValueError(f"RoLaQ artifact: {why}")
        model = manifest.get("model") or {}
        count = int(model["num_hidden_layers"])
        self.width = int(model["kv_lora_rank"])
        if set(manifest["layers"]) != {str(i) for i in range(count)}:
            raise ValueError("RoLaQ artifact must hold exactly one record per decoder layer")
        self.layers: dict[int, LayerRecord] = {}
        for key, item in manifest["layers"].items():
            layer = int(key)
            if item["file"] != f"layer_{layer}.pt":
                raise ValueError(f"layer {layer}: unexpected rotation file name {item['file']!r}")
            if file_sha256(self.root / item["file"]) != item["sha256"]:
                raise ValueError(f"layer {layer}: rotation file does not match its SHA-256")
            t, g = item["param0"], item["param1"]
            if not all(isinstance(v, (int, float)) and math.isfinite(v) and v > 0 for v in (t, g)):
                raise ValueError(f"layer {layer}: quantizer threshold/gain must be finite and positive")
            self.layers[layer] = LayerRecord(item["file"], item["sha256"], float(t), float(g))
        self.manifest = manifest

    def quantizer(self, layer: int) -> tuple[float, float]:
        rec = self.layers[int(layer)]
        return rec.threshold, rec.gain

    def rotation(self, layer: int, width: int | None = None) -> torch.Tensor:
        rec = self.layers[int(layer)]
        r = torch.load(self.root / rec.file, map_location="cpu", weights_only=True)
        return check_rotation(r, width if width is not None else self.width, layer)


@lru_cache(maxsize=8)
def open_artifact(path) -> Artifact:
    return Artifact(path)


def load_layer_quantizers(path, rotation_path, group_size, width, layer_ids):
    """Per-layer ``(threshold, gain)``; ``[None] * len(layer_ids)`` without an artifact."""
    if not path:
        return [None for _ in layer_ids]
    if Path(path).resolve() != Path(rotation_path).resolve():
        raise ValueError("the quantizer parameters and the rotations must come from one artifact")
    art = open_artifact(str(Path(path).resolve()))
    if group_size != GROUP_SIZE or art.width != width:
        raise ValueError("RoLaQ artifact does not match the cache's group size / latent width")
    return [art.quantizer(layer) for layer in layer_ids]


def load_rotation(rotation_path, layer_id: int, width: int | None = None) -> torch.Tensor:
    """The checked FP32 rotation of one layer (no manifest needed)."""
    r = torch.load(Path(rotation_path) / f"layer_{layer_id}.pt", map_location="cpu", weights_only=True)
    return check_rotation(r, width, layer_id)


def fold_read_rotation(weight, layer_id, rotation_path):
    """``bf16(W_b @ fp32(bf16(R)))`` for the absorbed MLA readers.

    ``W_b`` is ``[heads * (key_dim + value_dim), latent_dim]`` bf16. Queries and
    outputs of the absorbed path then live in the rotated frame, so the readers
    apply no rotation at run time. The product is formed in FP32 with the same
    effective rotation the writer uses (R rounded to bf16, read back as FP32).
    """
    if weight.dtype != torch.bfloat16:
        raise ValueError("read-rotation folding is defined for bf16 weights only")
    r = torch.load(Path(rotation_path) / f"layer_{layer_id}.pt", map_location="cpu", weights_only=True)
    if tuple(r.shape) != (weight.shape[-1], weight.shape[-1]):
        raise ValueError("read rotation does not match the weight's latent width")
    effective = r.to(device=weight.device, dtype=torch.bfloat16).float()
    return (weight.float() @ effective).to(torch.bfloat16)


def write_artifact(root, rotations: dict, params: dict, model: dict) -> dict:
    """Write an artifact directory in the reference's format (field names of
    mla_quant/quantizer.py:190-213); used to build test artifacts."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=False)
    layers = {}
    for layer in sorted(rotations):
        path = root / f"layer_{layer}.pt"
        torch.save(rotations[layer].detach().cpu().float().contiguous(), path)
        t, g = params[layer]
        layers[str(layer)] = {"file": path.name, "sha256": file_sha256(path), "param0": float(t), "param1": float(g)}
    manifest = {"format_version": FORMAT_VERSION, "recipe": RECIPE, "family": "oscar_lloyd",
                "group_size": GROUP_SIZE, "components": ["nope"], "windows": False, "model": dict(model),
                "layers": layers}
    (root / "manifest.json").write_text(json.dumps(manifest, indent=2))
    return manifest
