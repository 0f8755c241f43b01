"""Oracle: the OSCAR/RoLaQ Lloyd INT2 codec and its cast order.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates ``mla_quant/oscar.py:104-144`` (constants and the QDQ codec),
``mla_quant/quantizer.py:31-35`` (gain snapping), ``:102-124`` (cast order of
``rotate_quantize``), ``:145-152`` (rotation validation) and
``mla_quant/train.py:21-29`` (``signal_gain``), and ``kv_a_layernorm``: the
third-party ``DeepseekV2RMSNorm.forward`` (transformers 5.15.0,
``models/deepseek_v2/modeling_deepseek_v2.py:166-171``) whose output the
reference quantizes (``mla_quant/objectives.py:25-29``, ``calibrate.py:40``).
"""

from __future__ import annotations

import math

import numpy as np
import torch

# mla_quant/oscar.py:104-111 -- Lloyd-Max constants for a unit Gaussian.
LLOYD_MAX_THRESHOLD = 0.9810652732849121
LLOYD_MAX_CENTROIDS = (
    -1.5095585584640503,
    -0.4527800381183624,
    0.4527800381183624,
    1.5095585584640503,
)
LLOYD_MAX_STRETCH = 1.16
# oscar.py:141-143: the affine grid spans the outer centroids in 3 steps.
SPAN = LLOYD_MAX_CENTROIDS[3] - LLOYD_MAX_CENTROIDS[0]
SPAN3 = SPAN / 3.0
ZERO_OFFSET = -LLOYD_MAX_CENTROIDS[0] / SPAN3  # 1.5 exactly in float64
# oscar.py:112-117 -- the uniform reconstruction levels.
OSCAR_LLOYD_CENTERS = tuple(
    LLOYD_MAX_CENTROIDS[0] + i * (LLOYD_MAX_CENTROIDS[3] - LLOYD_MAX_CENTROIDS[0]) / 3
    for i in range(4)
)
# quantizer.py:26 -- admissible (threshold, gain) ranges.
LLOYD_BOUNDS = ((0.5, 1.5), (0.8, 1.3))
GROUP_SIZE = 128


def snap_gain(gain: float) -> float:
    """quantizer.py:31-35: an FP32-rounded 1.16 is replaced by the float64 1.16."""
    gain = float(gain)
    if gain == float(torch.tensor(LLOYD_MAX_STRETCH, dtype=torch.float32)):
        return LLOYD_MAX_STRETCH
    return gain


def scale_factor(gain: float) -> np.float32:
    """The FP32 constant multiplying ``std`` in ``scale`` (oscar.py:142).

    ``span / 3.0 * gain`` is a Python float product; torch then casts it to the
    tensor dtype (FP32) before multiplying by ``std``.
    """
    return np.float32(SPAN3 * float(gain))


def lloyd_codec(values: torch.Tensor, group_size: int = GROUP_SIZE,
                threshold: float = LLOYD_MAX_THRESHOLD, gain: float = LLOYD_MAX_STRETCH):
    """Restates ``oscar_lloyd_int2_qdq`` (mla_quant/oscar.py:120-144).

    Returns ``(codes, scale, zero, qdq)``: codes uint8 in 0..3 with the input's
    shape, ``scale``/``zero`` FP32 of shape ``[rows, D // group_size]`` and the
    FP32 fake-quantized values. The operation order is the reference's, in FP32
    on the CPU, so ``qdq`` equals the reference output bit for bit.
    """
    shape = values.shape
    width = shape[-1]
    if width % group_size:
        raise ValueError("width must be a multiple of the group size")
    groups = values.reshape(-1, group_size).float()
    mean = groups.mean(-1, keepdim=True)
    diff = groups - mean
    std = (diff.pow(2).mean(-1, keepdim=True) + 1e-08).sqrt()
    normalized = diff / std
    t = float(threshold)
    codes = ((normalized >= -t).to(torch.uint8) + (normalized >= 0.0).to(torch.uint8)
             + (normalized >= t).to(torch.uint8))
    scale = SPAN3 * float(gain) * std
    zero = ZERO_OFFSET - mean / scale
    qdq = (codes.float() - zero) * scale
    rows = groups.shape[0] * group_size // width
    ng = width // group_size
    return (codes.reshape(shape), scale.reshape(rows, ng), zero.reshape(rows, ng),
            qdq.reshape(shape))


def dequantize(codes: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor,
               group_size: int = GROUP_SIZE) -> torch.Tensor:
    """FP32 reconstruction ``(code - zero) * scale`` per group (oscar.py:144)."""
    rows, width = codes.shape
    ng = width // group_size
    c = codes.reshape(rows, ng, group_size).float()
    return ((c - zero.reshape(rows, ng, 1).float()) * scale.reshape(rows, ng, 1).float()).reshape(rows, width)


def effective_rotation(rotation: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    """quantizer.py:117 / rolaq_mla.py:69-70: FP32 -> model dtype -> FP32."""
    return rotation.to(dtype=dtype).float()


def rotate(latent: torch.Tensor, rotation: torch.Tensor) -> torch.Tensor:
    """quantizer.py:117-118: ``latent.float() @ R_eff`` in FP32."""
    return latent.float() @ effective_rotation(rotation, latent.dtype)


def rotate_quantize(latent: torch.Tensor, rotation: torch.Tensor,
                    threshold: float = LLOYD_MAX_THRESHOLD, gain: float = LLOYD_MAX_STRETCH,
                    high_precision_mask: torch.Tensor | None = None,
                    group_size: int = GROUP_SIZE) -> torch.Tensor:
    """Restates ``rotate_quantize`` (quantizer.py:102-124) for the Lloyd family.

    Rotate in FP32 with the bf16-rounded rotation, QDQ, round to the input
    dtype, rotate back in FP32 and round again. Rows flagged in
    ``high_precision_mask`` (shape ``latent.shape[:-1]``) are returned untouched.
    """
    if high_precision_mask is not None:
        mask = torch.broadcast_to(high_precision_mask.to(torch.bool), latent.shape[:-1])
        if bool(mask.all()):
            return latent
    effective = effective_rotation(rotation, latent.dtype)
    rotated = latent.float() @ effective
    _, _, _, quantized = lloyd_codec(rotated, group_size, threshold, snap_gain(gain))
    dequantized = quantized.to(dtype=latent.dtype)
    restored = (dequantized.float() @ effective.T).to(dtype=latent.dtype)
    if high_precision_mask is None:
        return restored
    return torch.where(mask.unsqueeze(-1), latent, restored)


def kv_a_layernorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMS norm with the cast order of DeepseekV2RMSNorm.forward (transformers
    5.15.0, models/deepseek_v2/modeling_deepseek_v2.py:166-171).

    Statistics in FP32 (``mean(x^2)`` over the last dim, ``rsqrt(var + eps)``),
    the normalized row rounded to the input dtype, then multiplied by the
    weight in the weight's dtype: ``bf16(w * bf16(x * r))`` for bf16 inputs.
    CPU torch ops (``rsqrt`` on CPU is ``1 / sqrt`` in FP32).
    """
    h = x.to(torch.float32)
    r = torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return weight * (h * r).to(x.dtype)


def signal_gain(threshold) -> float:
    """train.py:21-29: ``g(t) = 1 / (2 (|c1| (phi(0) - phi(t)) + |c3| phi(t)))``.

    ``phi(t)`` is evaluated in the threshold tensor's dtype (FP32 for a float
    tensor), as the reference does; returns a Python float.
    """
    t = torch.as_tensor(threshold, dtype=torch.float32)
    phi0 = 1 / math.sqrt(2 * math.pi)
    phi_t = torch.exp(-t.square() / 2) * phi0
    inner, outer = abs(OSCAR_LLOYD_CENTERS[1]), abs(OSCAR_LLOYD_CENTERS[3])
    return float(1 / (2 * (inner * (phi0 - phi_t) + outer * phi_t)))


def validate_rotation(rotation: torch.Tensor, width: int) -> None:
    """quantizer.py:145-152: square FP32, finite, orthogonal to 1e-5."""
    if rotation.dtype != torch.float32 or tuple(rotation.shape) != (width, width):
        raise ValueError("rotation must be a square FP32 matrix")
    if not torch.isfinite(rotation).all():
        raise ValueError("rotation contains non-finite values")
    residual = (rotation.double().T @ rotation.double() - torch.eye(width, dtype=torch.float64)).abs().max().item()
    if residual > 1e-05:
        raise ValueError(f"rotation not orthogonal, residual={residual}")


def validate_parameters(threshold: float, gain: float) -> None:
    """quantizer.py:136-142: finite and within LLOYD_BOUNDS (1e-6 slack)."""
    for value, (lo, hi) in zip((threshold, gain), LLOYD_BOUNDS):
        if not math.isfinite(value) or not lo - 1e-06 <= value <= hi + 1e-06:
            raise ValueError("quantizer parameter non-finite or out of bounds")
