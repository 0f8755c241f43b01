"""Pin the oracle's Lloyd INT2 codec (CPU only)."""

import math

import numpy as np
import pytest
import torch

from oracle import codec
from mla_kv_quant_amd import synth

K_DEFAULT = np.float32(1.1673918962478638)  # fp32(span/3 * 1.16)


def test_constants_closed_form():
    c = codec.LLOYD_MAX_CENTROIDS
    assert codec.SPAN == pytest.approx(2 * c[3])
    assert codec.ZERO_OFFSET == 1.5
    assert codec.scale_factor(1.16) == K_DEFAULT
    assert float(np.float32(codec.LLOYD_MAX_THRESHOLD)) == codec.LLOYD_MAX_THRESHOLD
    # uniform reconstruction grid: centers are equally spaced over the outer centroids
    centers = codec.OSCAR_LLOYD_CENTERS
    steps = np.diff(centers)
    assert np.allclose(steps, codec.SPAN3)


@pytest.mark.parametrize("case", [0, 1, 2])
def test_codec_matches_reference_golden(golden_dir, case):
    g = np.load(golden_dir / "codec_golden.npz")
    values = torch.from_numpy(g["values"])
    t, gain = float(g[f"t{case}"]), float(g[f"g{case}"])
    _, _, _, qdq = codec.lloyd_codec(values, 128, t, gain)
    ref = g[f"qdq{case}"]
    assert qdq.numpy().view(np.uint32).tobytes() == ref.view(np.uint32).tobytes()


def test_constant_group_special_case():
    x = torch.full((1, 128), 3.25)
    codes, scale, zero, qdq = codec.lloyd_codec(x)
    std = np.sqrt(np.float32(1e-8))
    assert (codes == 2).all()
    assert scale.item() == pytest.approx(float(K_DEFAULT * std), rel=1e-6)
    assert torch.allclose(qdq, torch.full_like(qdq, 3.25 + 0.5 * scale.item()), rtol=0, atol=1e-6)


@pytest.mark.parametrize("t,expect", [(0.9810652732849121, (3, 0)), (1.2, (2, 1))])
def test_alternating_group_closed_form(t, expect):
    x = torch.empty(1, 128)
    x[0, ::2], x[0, 1::2] = 1.0, -1.0
    codes, scale, zero, qdq = codec.lloyd_codec(x, 128, t, 1.16)
    assert (codes[0, ::2] == expect[0]).all() and (codes[0, 1::2] == expect[1]).all()
    # biased variance: std = sqrt(1 + 1e-8) == 1 in fp32, so scale == K, zero == 1.5
    assert scale.item() == float(K_DEFAULT)
    assert zero.item() == 1.5
    k = float(K_DEFAULT)
    assert qdq[0, 0].item() == pytest.approx((expect[0] - 1.5) * k, abs=1e-6)
    assert qdq[0, 1].item() == pytest.approx((expect[1] - 1.5) * k, abs=1e-6)


def test_four_levels_monotone_and_recoverable():
    x = synth.make_latent(64, 512, 5, seed=3).float()
    codes, scale, zero, qdq = codec.lloyd_codec(x)
    groups = x.reshape(64, 4, 128)
    cg = codes.reshape(64, 4, 128)
    # codes are monotone in the value inside each group
    order = groups.argsort(-1)
    sorted_codes = torch.gather(cg, -1, order)
    assert (sorted_codes[..., 1:] >= sorted_codes[..., :-1]).all()
    # every reconstruction is one of mean + (k - 1.5) * scale
    mean = groups.mean(-1)
    levels = mean[..., None] + (torch.arange(4).float() - 1.5) * scale[..., None]
    recon = qdq.reshape(64, 4, 128)
    picked = torch.gather(levels, -1, cg.long())
    assert torch.allclose(recon, picked, rtol=0, atol=1e-5 * scale.max().item())
    # codes are recoverable from the QDQ output and the params
    back = torch.round(recon / scale[..., None] + zero[..., None])
    assert torch.equal(back.to(torch.uint8), cg)
    # dequantize() is the same reconstruction
    assert torch.equal(codec.dequantize(codes, scale, zero), qdq)


def test_gain_snapping_and_bounds():
    assert codec.snap_gain(float(np.float32(1.16))) == 1.16
    assert codec.snap_gain(1.2) == 1.2
    codec.validate_parameters(0.98, 1.16)
    with pytest.raises(ValueError):
        codec.validate_parameters(1.6, 1.16)
    with pytest.raises(ValueError):
        codec.validate_parameters(0.9, float("nan"))


def test_signal_gain_closed_form():
    c1, c3 = codec.OSCAR_LLOYD_CENTERS[1], codec.OSCAR_LLOYD_CENTERS[3]

    def g64(t):
        phi0 = 1 / math.sqrt(2 * math.pi)
        phit = math.exp(-t * t / 2) * phi0
        return 1 / (2 * (abs(c1) * (phi0 - phit) + abs(c3) * phit))

    for t in (0.5, 0.75, 0.9810652732849121, 1.2):
        assert codec.signal_gain(t) == pytest.approx(g64(t), rel=2e-6)
    # g(t) crosses the upper gain bound 1.3 near t = 1.2497
    assert codec.signal_gain(1.2497) < 1.3 < codec.signal_gain(1.2498)
    # at t -> 0 the response is 2 |c3| phi(0): g(0) = 1 / (2 |c3| phi0)
    assert codec.signal_gain(0.0) == pytest.approx(1 / (2 * abs(c3) / math.sqrt(2 * math.pi)), rel=1e-6)
    # learned-style generator uses the same law
    for t, g in synth.learned_style_params(5, 1):
        assert g == pytest.approx(codec.signal_gain(t), rel=1e-6)


def test_rotate_quantize_matches_reference_golden(golden_dir):
    import hashlib
    g = np.load(golden_dir / "rotate_quantize_golden.npz")
    for width in (512, 256):
        r = synth.make_rotation(width, int(g[f"seed{width}"]))
        sha = hashlib.sha256(r.numpy().tobytes()).hexdigest()
        if sha != bytes(g[f"sha{width}"]).decode():
            pytest.skip("this host's LAPACK QR does not reproduce the fixture rotation bit for bit")
        x = torch.from_numpy(g[f"x{width}"]).view(torch.bfloat16)
        mask = torch.from_numpy(g[f"mask{width}"])
        y = codec.rotate_quantize(x, r)
        ym = codec.rotate_quantize(x, r, high_precision_mask=mask)
        assert torch.equal(y.view(torch.int16), torch.from_numpy(g[f"y{width}"]))
        assert torch.equal(ym.view(torch.int16), torch.from_numpy(g[f"ym{width}"]))


def test_rotation_validator_and_cast_order():
    r = synth.make_rotation(256, 7)
    codec.validate_rotation(r, 256)
    with pytest.raises(ValueError):
        codec.validate_rotation(r * 1.01, 256)
    with pytest.raises(ValueError):
        codec.validate_rotation(r.double(), 256)
    # the effective rotation is exactly bf16-representable (bf16 products are exact)
    eff = codec.effective_rotation(r)
    assert torch.equal(eff, eff.to(torch.bfloat16).float())
    # rotate-quantize-unrotate with an all-BF16 mask is the identity
    x = synth.make_latent(3, 256, 0, seed=1)
    assert torch.equal(codec.rotate_quantize(x, r, high_precision_mask=torch.ones(3, dtype=torch.bool)), x)
