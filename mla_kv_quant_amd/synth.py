"""Seeded synthetic inputs at the benchmark shapes.

There is no network and no checkpoint: the latent rows, RoPE keys, queries and
rotations are synthetic, drawn with ``torch.Generator().manual_seed(seed)`` so
that every test and benchmark is reproducible.
"""

from __future__ import annotations

import math

import torch

# OSCAR default quantizer (mla_quant/oscar.py:104,111).
DEFAULT_THRESHOLD = 0.9810652732849121
DEFAULT_GAIN = 1.16


def make_rotation(width: int, seed: int) -> torch.Tensor:
    """Orthogonal FP32 ``[width, width]``: ``Q diag(sign(diag(R)))`` from the QR
    of a float64 Gaussian (the rotation validator's 1e-5 residual holds)."""
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(width, width, generator=g, dtype=torch.float64)
    q, r = torch.linalg.qr(a)
    q = q * torch.sign(torch.diagonal(r))[None, :]
    return q.float().contiguous()


def layer_rotation(width: int, layer: int) -> torch.Tensor:
    """Rotation of layer ``layer`` (seed ``1000 + layer``)."""
    return make_rotation(width, 1000 + layer)


def outlier_channels(width: int, count: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(width, generator=g)[:count]


def make_latent(n: int, width: int, outliers: int, seed: int, factor: float = 20.0,
                device="cpu") -> torch.Tensor:
    """bf16 ``[n, width]`` N(0,1) rows whose ``outliers`` channels are scaled by
    ``factor`` before the bf16 cast."""
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(n, width, generator=g, device=device, dtype=torch.float32)
    if outliers:
        ch = outlier_channels(width, outliers, seed + 7).to(device)
        x[:, ch] *= factor
    return x.to(torch.bfloat16)


def make_kv_a(n: int, width: int, seed: int, device="cpu") -> torch.Tensor:
    """bf16 pre-norm compressed latents ``kv_a``: N(0, 0.05^2) rows with a few
    channels x20, and per-row magnitudes spread over two octaves."""
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(n, width, generator=g, device=device, dtype=torch.float32) * 0.05
    ch = outlier_channels(width, max(1, width // 100), seed + 7).to(device)
    x[:, ch] *= 20.0
    x *= torch.exp2(torch.rand(n, 1, generator=g, device=device) * 2.0 - 1.0)
    return x.to(torch.bfloat16)


def make_norm_weight(width: int, seed: int, device="cpu") -> torch.Tensor:
    """bf16 ``kv_a_layernorm`` weight: |N(1, 0.3^2)| with a few channels x8
    (the post-norm latent's outlier channels come from the weight)."""
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(width, generator=g) * 0.3 + 1.0).abs()
    w[outlier_channels(width, max(1, width // 100), seed + 3)] *= 8.0
    return w.to(torch.bfloat16).to(device)


def make_normal(shape, seed: int, std: float = 1.0, device="cpu",
                dtype=torch.bfloat16) -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std).to(dtype)


def learned_style_params(layers: int, seed: int):
    """RoLaQ-style per-layer ``(t, g(t))`` with ``t ~ U[0.6, 1.2]`` (train.py:21-29)."""
    g = torch.Generator().manual_seed(seed)
    t = (torch.rand(layers, generator=g) * 0.6 + 0.6).float()
    out = []
    for i in range(layers):
        ti = t[i]
        phi0 = 1 / math.sqrt(2 * math.pi)
        phi_t = torch.exp(-ti.square() / 2) * phi0
        c = (-1.5095585584640503, 1.5095585584640503)
        inner = abs(c[0] + (c[1] - c[0]) / 3)
        outer = abs(c[1])
        gain = float(1 / (2 * (inner * (phi0 - phi_t) + outer * phi_t)))
        out.append((float(ti), gain))
    return out
