"""GPU parity: quantize-dequantize of latent rows (``rotate_quantize``) against the CPU oracle.

Oracle: ``oracle.codec.rotate_quantize`` (restates mla_quant/quantizer.py:102-124).
The GPU forms the same products (bf16-exact operands, FP32 accumulation) in a
different summation order, so a code can flip by one level at a rounding
boundary (the writer's budget: <= 1e-5 of the elements). A row without a flip
must match to one bf16 unit in the last place (both sides round an FP32 value
that differs only in its last bits); a flipped row moves by at most one
quantization level in the rotated frame.
"""

import numpy as np
import pytest
import torch

from oracle import codec
from mla_kv_quant_amd import qdq, synth

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _compare(gpu: torch.Tensor, ref: torch.Tensor, flip_budget: float):
    g, r = gpu.float().reshape(-1, gpu.shape[-1]), ref.float().reshape(-1, ref.shape[-1])
    ulp = torch.clamp(r.abs(), min=2.0 ** -120) * 2.0 ** -7  # >= one bf16 ulp of the reference
    bad_rows = ((g - r).abs() > ulp).any(-1)
    nbad = int(bad_rows.sum())
    assert nbad <= max(2, flip_budget * g.numel()), f"{nbad} rows differ by more than one bf16 ulp"
    return nbad


@pytest.mark.parametrize("D", [512, 256])
@pytest.mark.parametrize("tg", [(qdq.LM_THRESHOLD, qdq.LM_GAIN), (0.8, None)])
def test_rotate_quantize_matches_oracle(D, tg):
    t, g = tg
    g = codec.signal_gain(t) if g is None else g
    x = synth.make_latent(3 * 700, D, max(1, D // 100), seed=D + 1).reshape(3, 700, D)
    rot = synth.make_rotation(D, 7)
    ref = codec.rotate_quantize(x, rot, t, g)
    out = qdq.rotate_quantize(x.to(DEV), rot, t, g)
    torch.cuda.synchronize()
    assert out.shape == x.shape and out.dtype == torch.bfloat16
    _compare(out.cpu(), ref, 1e-5)


def test_rotate_quantize_mask_and_edges():
    D = 512
    x = synth.make_latent(2 * 40, D, 5, seed=3).reshape(2, 40, D)
    rot = synth.make_rotation(D, 8)
    mask = torch.zeros(2, 40, dtype=torch.bool)
    mask[:, :4] = True          # sink rows
    mask[1, -16:] = True        # recent rows of the second sequence
    ref = codec.rotate_quantize(x, rot, high_precision_mask=mask)
    out = qdq.rotate_quantize(x.to(DEV), rot, high_precision_mask=mask.to(DEV)).cpu()
    assert torch.equal(out[mask], x[mask])            # flagged rows untouched
    _compare(out, ref, 1e-5)
    # every row flagged: the input itself; no rows: an empty result
    xd = x.to(DEV)
    assert qdq.rotate_quantize(xd, rot, high_precision_mask=torch.ones(2, 40, dtype=torch.bool)) is xd
    assert qdq.rotate_quantize(xd[:, :0], rot).shape == (2, 0, D)
    with pytest.raises(ValueError):
        qdq.rotate_quantize(xd.float(), rot)
    with pytest.raises(ValueError):
        qdq.rotate_quantize(xd, rot[:256, :256].contiguous())
    with pytest.raises(ValueError):
        qdq.rotate_quantize(xd, rot, group_size=64)
