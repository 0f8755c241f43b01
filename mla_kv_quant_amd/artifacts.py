"""RoLaQ artifact loader and read-rotation folding (host side).

Restates deployment/sglang/srt/mem_cache/rolaq_mla.py:16-71 (manifest checks,
per-layer ``(threshold, gain)``, ``W_b @ fp32(bf16(R))``) with the rotation
checks of mla_quant/quantizer.py:145-152. An artifact is a directory holding
``manifest.json`` and ``layer_<i>.pt`` (FP32 ``[D, D]`` rotations), loaded with
``torch.load(..., weights_only=True)``.
"""

from __future__ import annotations

import hashlib
import json
import math
from functools import lru_cache
from pathlib import Path

import torch

RECIPE = "learned_shared_latent_rotation_quantizer_v2"
FORMAT_VERSION = 2


def _sha256(path: Path) -> str:
    h = hashlib.sha256()
    with path.open("rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


@lru_cache(maxsize=8)
def load_manifest(path):
    """Validate and return the manifest (rolaq_mla.py:16-38)."""
    root = Path(path).resolve()
    manifest = json.loads((root / "manifest.json").read_text())
    if manifest.get("recipe") != RECIPE:
        raise ValueError("RoLaQ requires a frozen v2 learned artifact")
    if manifest.get("family") != "oscar_lloyd":
        raise ValueError("The packed RoLaQ writer currently supports oscar_lloyd only")
    if manifest.get("components") != ["nope"] or manifest.get("group_size") != 128:
        raise ValueError("Expected content-only, group-128 RoLaQ artifact")
    count = manifest["model"]["num_hidden_layers"]
    if set(manifest["layers"]) != {str(i) for i in range(count)}:
        raise ValueError("RoLaQ artifact must cover every decoder layer")
    for layer, item in manifest["layers"].items():
        if item["file"] != f"layer_{int(layer)}.pt":
            raise ValueError("Unexpected rotation filename")
        if _sha256(root / item["file"]) != item["sha256"]:
            raise ValueError(f"RoLaQ rotation hash mismatch: layer {layer}")
        t, gain = item["param0"], item["param1"]
        if not (math.isfinite(t) and math.isfinite(gain) and t > 0 and gain > 0):
            raise ValueError(f"Invalid quantizer parameters at layer {layer}")
    return manifest


def load_layer_quantizers(path, rotation_path, group_size, width, layer_ids):
    """Per-layer ``(threshold, gain)`` or ``None`` without an artifact (rolaq_mla.py:41-53)."""
    if not path:
        return [None for _ in layer_ids]
    if Path(path).resolve() != Path(rotation_path).resolve():
        raise ValueError("Learned quantizer and rotations must come from the same artifact")
    manifest = load_manifest(path)
    if manifest["group_size"] != group_size or manifest["model"]["kv_lora_rank"] != width:
        raise ValueError("RoLaQ artifact does not match the cache dimensions")
    out = []
    for layer in layer_ids:
        item = manifest["layers"][str(layer)]
        out.append((float(item["param0"]), float(item["param1"])))
    return out


def load_rotation(rotation_path, layer_id: int, width: int | None = None) -> torch.Tensor:
    """FP32 rotation of one layer, checked square/finite/orthogonal (quantizer.py:145-152)."""
    rotation = torch.load(Path(rotation_path) / f"layer_{layer_id}.pt", map_location="cpu", weights_only=True)
    if not isinstance(rotation, torch.Tensor) or rotation.dtype != torch.float32 or rotation.dim() != 2 \
            or rotation.shape[0] != rotation.shape[1] or (width is not None and rotation.shape[0] != width):
        raise ValueError(f"layer {layer_id} requires a square FP32 rotation")
    if not torch.isfinite(rotation).all():
        raise ValueError(f"layer {layer_id} rotation contains non-finite values")
    n = rotation.shape[0]
    residual = (rotation.double().T @ rotation.double() - torch.eye(n, dtype=torch.float64)).abs().max().item()
    if residual > 1e-05:
        raise ValueError(f"layer {layer_id} rotation not orthogonal, residual={residual}")
    return rotation


def fold_read_rotation(weight, layer_id, rotation_path):
    """Return ``W_b @ R`` for derived MLA readers (rolaq_mla.py:56-71).

    ``W_b`` is ``[heads * (key_dim + value_dim), latent_dim]`` bf16; the product
    is formed in FP32 with ``R_eff = fp32(bf16(R))`` and rounded to bf16.
    """
    if weight.dtype != torch.bfloat16:
        raise ValueError("Read-rotation absorption is validated for BF16 weights only")
    rotation = torch.load(Path(rotation_path) / f"layer_{layer_id}.pt", map_location="cpu", weights_only=True)
    if rotation.shape != (weight.shape[-1], weight.shape[-1]):
        raise ValueError("Read-rotation shape mismatch")
    effective = rotation.to(device=weight.device, dtype=weight.dtype).float()
    return (weight.float() @ effective).to(weight.dtype)


def write_artifact(root, rotations: dict, params: dict, model: dict) -> dict:
    """Write a manifest + per-layer rotations in the reference's artifact format
    (mla_quant/quantizer.py:155-215 field names); used to build test artifacts."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=False)
    layers = {}
    for layer in sorted(rotations):
        path = root / f"layer_{layer}.pt"
        torch.save(rotations[layer].detach().cpu().float().contiguous(), path)
        t, g = params[layer]
        layers[str(layer)] = {"file": path.name, "sha256": _sha256(path), "param0": float(t), "param1": float(g)}
    manifest = {"format_version": FORMAT_VERSION, "recipe": RECIPE, "family": "oscar_lloyd",
                "group_size": 128, "components": ["nope"], "windows": False, "model": dict(model),
                "layers": layers}
    (root / "manifest.json").write_text(json.dumps(manifest, indent=2))
    return manifest
