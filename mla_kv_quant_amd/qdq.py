"""GPU quantize-dequantize of latent rows (the HF fake-quantized cache path).

``rotate_quantize`` mirrors mla_quant/quantizer.py:102-124 (name, arguments,
cast order): rotate in FP32 with ``R_eff = fp32(bf16(R))``, Lloyd INT2 QDQ per
group of 128, round to the input dtype, rotate back in FP32 and round again;
rows flagged in ``high_precision_mask`` come back untouched. The reference's
``FakeQuantizedDynamicCache`` (mla_quant/cache.py:683-1118) applies it to every
cached latent row on update; here it runs as two launches of this library's
kernels instead of torch CPU/GPU ops:

1. the fused writer (rotation on bf16 MFMA with FP32 accumulation -- both
   operands are bf16-exact -- then the quantizer) into scratch codes/params;
2. the dequantize-rows kernel with un-rotation: ``(code - zero) * scale``
   rounded to bf16, times ``R_eff^T`` in FP32, rounded to bf16.

Only the summation order differs from the reference, so codes agree except for
rare +-1 flips at rounding boundaries (the writer's parity bar).

``LearnedRotationQuantizer`` is the GPU counterpart of the reference's
inference quantizer of the same name (mla_quant/quantizer.py:218-316): built
from an artifact directory, ``quantize_layer(tensor, layer_idx, "nope")`` is
what the HF fake-quantized cache calls for every appended latent row
(``FakeQuantizedDynamicCache._quantize_component``, mla_quant/cache.py:802-816),
so passing an instance as that cache's ``quantizer`` runs the evaluation's QDQ
through these kernels.
"""

from __future__ import annotations

import torch

from . import kernels
from .artifacts import Artifact
from .writer import LM_GAIN, LM_THRESHOLD, SUPPORTED_DIMS

GROUP_SIZE = 128

# Read-only helper tensors per (device, D), grown to the largest row count
# seen: the slot ids 1..n, seq_len 1, request 0, zero rope keys and an empty
# window. The writer writes row_of_slot[slot] = -1 for these rows (no window:
# P = W = 0), the value it already holds, so sharing them across calls and
# streams is safe.
_HELPERS: dict = {}


# bf16 R_eff and its transpose on the device, per rotation tensor (held, so
# its id stays unique) and its version counter (an in-place update re-derives).
_ROTATIONS: dict = {}


def _rotation_operands(rotation: torch.Tensor, dev: torch.device):
    key = (id(rotation), rotation._version, str(dev))
    hit = _ROTATIONS.get(key)
    if hit is None:
        r_eff = rotation.to(device=dev, dtype=torch.bfloat16).contiguous()
        if len(_ROTATIONS) >= 16:
            _ROTATIONS.pop(next(iter(_ROTATIONS)))
        hit = _ROTATIONS[key] = (rotation, r_eff, r_eff.t().contiguous())
    return hit[1], hit[2]


def _helpers(dev: torch.device, n: int, D: int, R: int):
    key = (str(dev), D)
    h = _HELPERS.get(key)
    if h is None or h["cap"] < n:
        cap = max(n, 2 * h["cap"] if h else 0)
        h = _HELPERS[key] = {
            "cap": cap,
            "slots": torch.arange(1, cap + 1, dtype=torch.int64, device=dev),
            "ones": torch.ones(cap, dtype=torch.int64, device=dev),
            "zeros": torch.zeros(cap, dtype=torch.int64, device=dev),
            "pe": torch.zeros(cap, R, dtype=torch.bfloat16, device=dev),
            "row": torch.full((cap + 1,), -1, dtype=torch.int32, device=dev),
            "hp": torch.empty(1, D, dtype=torch.bfloat16, device=dev),
            "owner": torch.zeros(1, dtype=torch.int32, device=dev),
        }
    return h


def _normalize_mask(mask: torch.Tensor, latent: torch.Tensor) -> torch.Tensor:
    """``[seq]``, ``[batch, seq]`` or ``latent.shape[:-1]`` (``[batch, 1, seq]``)
    to ``latent.shape[:-1]`` (mla_quant/quantizer.py:85-99)."""
    mask = mask.to(device=latent.device, dtype=torch.bool)
    expected = tuple(latent.shape[:-1])
    if mask.ndim == 1 and len(expected) > 1:
        mask = mask.reshape(*[1] * (len(expected) - 1), mask.shape[0])
    elif mask.ndim == 2 and len(expected) == 3:
        mask = mask.unsqueeze(1)
    try:
        return torch.broadcast_to(mask, expected)
    except RuntimeError as error:
        raise ValueError(f"high precision mask shape {tuple(mask.shape)} does not match {expected}") from error


def rotate_quantize(latent: torch.Tensor, rotation: torch.Tensor, threshold: float = LM_THRESHOLD,
                    gain: float = LM_GAIN, high_precision_mask: torch.Tensor | None = None,
                    group_size: int = GROUP_SIZE) -> torch.Tensor:
    """Restored bf16 ``latent`` (any leading shape, last dim D) after rotate -> QDQ -> un-rotate.

    ``latent`` must be bf16 on the GPU and ``rotation`` a ``[D, D]`` FP32
    matrix; ``threshold``/``gain`` are the layer's Lloyd parameters.
    """
    if group_size != GROUP_SIZE:
        raise ValueError("the packed INT2 path quantizes groups of 128")
    if latent.dtype != torch.bfloat16 or not latent.is_cuda:
        raise ValueError("latent must be a bf16 GPU tensor")
    D = latent.shape[-1]
    R = 16 * (D // GROUP_SIZE)  # rope width the kernels are built for at this D
    if (D, R) not in SUPPORTED_DIMS:
        raise ValueError(f"unsupported latent width {D}")
    if rotation.dtype != torch.float32 or tuple(rotation.shape) != (D, D):
        raise ValueError("rotation must be a [D, D] FP32 matrix")
    mask = None
    if high_precision_mask is not None:
        mask = _normalize_mask(high_precision_mask, latent)
        if bool(mask.all()):
            return latent
    dev = latent.device
    x = latent.reshape(-1, D).contiguous()
    n = x.shape[0]
    if n == 0:
        return latent.clone()
    r_eff, r_eff_t = _rotation_operands(rotation, dev)
    h = _helpers(dev, n, D, R)
    slots = h["slots"][:n]
    # scratch cache: slots 1..n (slot 0 is the padding slot), no BF16 window
    codes = torch.empty(n + 1, D // 4, dtype=torch.uint8, device=dev)
    params = torch.empty(n + 1, D // GROUP_SIZE, 2, dtype=torch.float32, device=dev)
    rope = torch.empty(n + 1, R, dtype=torch.bfloat16, device=dev)
    kernels.write_rows(x, h["pe"][:n], r_eff_t, slots, h["ones"][:n], None, h["zeros"][:n], codes,
                       params, rope, h["hp"], h["row"][:n + 1], h["owner"], 0, 0, 1, float(threshold), float(gain))
    out = torch.empty(n, D + R, dtype=torch.bfloat16, device=dev)
    kernels.assemble_rows(slots, codes, params, rope, h["hp"], h["row"][:n + 1], h["owner"], r_eff, out)
    restored = out[:, :D].reshape(latent.shape)
    if mask is None:
        return restored
    return torch.where(mask.unsqueeze(-1), latent, restored)


# quantizer.py:31-35: a gain equal to FP32(1.16) is taken as the float64 1.16
_FP32_STRETCH = float(torch.tensor(LM_GAIN, dtype=torch.float32))


class LearnedRotationQuantizer:
    """GPU inference quantizer over a RoLaQ artifact (mla_quant/quantizer.py:218-316).

    Same construction checks (through :class:`Artifact`: manifest schema, every
    layer, SHA-256 of each rotation, orthogonality, parameter ranges), same
    ``quantize_layer`` contract and ``ValueError`` cases, same call counters
    and ``high_precision_mask`` handling (the last ``T`` positions of the mask
    for a ``T``-row append). The latent must be a bf16 GPU tensor -- the
    model's own dtype on this path. ``validate_config`` checks the model fields
    the manifest records; the checkpoint fingerprint the reference also
    compares needs the checkpoint files and is not checked here.
    """

    def __init__(self, artifact_dir):
        self.artifact = Artifact(artifact_dir)
        self.root = self.artifact.root
        self.manifest = self.artifact.manifest
        self.family = self.manifest["family"]
        self.width = self.artifact.width
        self.group_size = GROUP_SIZE
        self.rotations = {layer: self.artifact.rotation(layer) for layer in self.artifact.layers}
        self.params = {layer: self.artifact.quantizer(layer) for layer in self.artifact.layers}
        self.high_precision_mask: torch.Tensor | None = None
        self.layer_calls = {str(i): {"prefill": 0, "decode": 0} for i in self.rotations}
        self.call_count = 0
        self.element_count = 0
        self.first_shapes: list[tuple[int, ...]] = []

    def validate_config(self, config) -> None:
        expected = self.manifest.get("model", {})
        for key in ("model_type", "num_hidden_layers", "kv_lora_rank", "qk_rope_head_dim"):
            if key in expected and getattr(config, key, None) != expected[key]:
                raise ValueError(f"learned artifact model mismatch: {key}")

    def quantize_layer(self, tensor: torch.Tensor, layer_idx: int, component: str) -> torch.Tensor:
        if component != "nope":
            raise ValueError("learned rotation quantizes nope only")
        if tensor.ndim < 2 or tensor.shape[-1] != self.width or not tensor.is_floating_point():
            raise ValueError("invalid MLA latent shape or dtype")
        if layer_idx not in self.rotations:
            raise ValueError(f"missing learned rotation for layer {layer_idx}")
        phase = "decode" if tensor.shape[-2] == 1 else "prefill"
        self.layer_calls[str(layer_idx)][phase] += 1
        self.call_count += 1
        self.element_count += tensor.numel()
        if len(self.first_shapes) < 4:
            self.first_shapes.append(tuple(tensor.shape))
        t, g = self.params[layer_idx]
        t, g = float(torch.tensor(t, dtype=torch.float32)), float(torch.tensor(g, dtype=torch.float32))
        if g == _FP32_STRETCH:
            g = LM_GAIN
        mask = self.high_precision_mask
        if mask is not None and mask.shape[-1] != tensor.shape[-2]:
            mask = mask[..., -tensor.shape[-2]:]
        return rotate_quantize(tensor, self.rotations[layer_idx], t, g, high_precision_mask=mask)

    def metadata(self) -> dict:
        return {
            "recipe": self.manifest["recipe"],
            "family": self.family,
            "rotation_dir": str(self.root),
            "rotation_hashes": {str(k): v.sha256 for k, v in self.artifact.layers.items()},
            "components": ["nope"],
            "backend": "librolaq_mla (HIP, gfx950)",
        }
