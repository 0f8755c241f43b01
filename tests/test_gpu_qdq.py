"""GPU parity: quantize-dequantize of latent rows (``rotate_quantize``) against the CPU oracle.

Oracle: ``oracle.codec.rotate_quantize`` (restates mla_quant/quantizer.py:102-124).
The GPU forms the same products (bf16-exact operands, FP32 accumulation) in a
different summation order, so a code can flip by one level at a rounding
boundary (the writer's budget: <= 1e-5 of the elements). A row without a flip
must match to one bf16 unit in the last place (both sides round an FP32 value
that differs only in its last bits) -- or, for an element near zero where the
un-rotation's sum cancels, to 2^-16 of the row's largest magnitude (the FP32
summation-order error of a D-term sum); a flipped row moves by at most one
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
    # one bf16 ulp of the reference, and for elements near zero (where the
    # un-rotation's sum cancels) the FP32 summation-order error of a
    # D-term row, about 2^-16 of the row's largest magnitude
    tol = torch.maximum(r.abs() * 2.0 ** -7, r.abs().amax(-1, keepdim=True) * 2.0 ** -16)
    bad_rows = ((g - r).abs() > tol).any(-1)
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


def test_learned_rotation_quantizer_on_gpu(tmp_path):
    """quantize_layer through the GPU path equals the oracle's rotate_quantize
    with the artifact's parameters (FP32-rounded, gain 1.16 snapped as
    mla_quant/quantizer.py:31-35 does), including the high-precision mask."""
    from mla_kv_quant_amd import artifacts
    from mla_kv_quant_amd.qdq import LearnedRotationQuantizer

    D = 512
    rots = {i: synth.make_rotation(D, 40 + i) for i in range(2)}
    params = {0: (0.9, float(torch.tensor(1.16, dtype=torch.float32))), 1: (0.7, codec.signal_gain(0.7))}
    root = tmp_path / "art"
    artifacts.write_artifact(root, rots, params, {"model_type": "deepseek_v2", "num_hidden_layers": 2,
                                                  "kv_lora_rank": D, "qk_rope_head_dim": 64})
    q = LearnedRotationQuantizer(root)
    x = synth.make_latent(2 * 300, D, 5, seed=12).reshape(2, 1, 300, D)
    for layer in (0, 1):
        t, g = params[layer]
        t = float(torch.tensor(t, dtype=torch.float32))
        g = float(torch.tensor(g, dtype=torch.float32))
        g = 1.16 if g == float(torch.tensor(1.16, dtype=torch.float32)) else g
        ref = codec.rotate_quantize(x, rots[layer], t, g)
        out = q.quantize_layer(x.to(DEV), layer, "nope")
        torch.cuda.synchronize()
        _compare(out.cpu(), ref, 1e-5)
    # decode append with a [B, L] mask: its last T positions apply
    mask = torch.zeros(2, 40, dtype=torch.bool)
    mask[:, -2:] = True
    q.high_precision_mask = mask.to(DEV)
    x1 = synth.make_latent(2 * 4, D, 5, seed=13).reshape(2, 1, 4, D)
    out = q.quantize_layer(x1.to(DEV), 1, "nope").cpu()
    assert torch.equal(out[..., -2:, :], x1[..., -2:, :])
    t1 = float(torch.tensor(0.7, dtype=torch.float32))
    g1 = float(torch.tensor(codec.signal_gain(0.7), dtype=torch.float32))
    ref = codec.rotate_quantize(x1, rots[1], t1, g1)
    _compare(out[..., :2, :], ref[..., :2, :], 1e-5)
    assert q.layer_calls["1"] == {"prefill": 2, "decode": 0} and q.call_count == 3
