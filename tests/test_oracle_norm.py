"""Oracle pin: ``kv_a_layernorm`` against the third-party module it restates.

``oracle.codec.kv_a_layernorm`` restates DeepseekV2RMSNorm.forward
(transformers 5.15.0, models/deepseek_v2/modeling_deepseek_v2.py:166-171).
Pinned against that module itself (bit-exact on CPU) and against what the
mathematics fixes: exact invariance to power-of-two input scaling when
eps = 0, unit RMS of the output with a unit weight, and the weight applied
per column after the row's normalization.
"""

import pytest
import torch

from mla_kv_quant_amd import synth
from oracle import codec


@pytest.mark.parametrize("D", [512, 256])
def test_matches_transformers_deepseek_v2_rmsnorm(D):
    mod = pytest.importorskip("transformers.models.deepseek_v2.modeling_deepseek_v2")
    norm = mod.DeepseekV2RMSNorm(D, eps=1e-6).to(torch.bfloat16)
    w = synth.make_norm_weight(D, 4)
    with torch.no_grad():
        norm.weight.copy_(w)
    x = synth.make_kv_a(2000, D, 11)
    x[0] = 0.0                                  # all-zero row: eps keeps it finite
    x[1] = 3.0e4                                # large constant row
    with torch.no_grad():
        ref = norm(x)
    got = codec.kv_a_layernorm(x, w, 1e-6)
    assert got.dtype == ref.dtype == torch.bfloat16
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert not got[0].any()


def test_norm_invariants():
    D = 512
    x = synth.make_kv_a(500, D, 12)
    ones = torch.ones(D, dtype=torch.bfloat16)
    y = codec.kv_a_layernorm(x, ones, 0.0)
    # eps = 0: scaling by a power of two leaves the result bit-identical
    assert torch.equal(codec.kv_a_layernorm(x * 8, ones, 0.0), y)
    assert torch.equal(codec.kv_a_layernorm(x / 4, ones, 0.0), y)
    # unit weight: every row has unit RMS up to the bf16 rounding of its elements
    rms = y.float().pow(2).mean(-1).sqrt()
    assert torch.all((rms - 1).abs() < 2 ** -8)
    # the weight multiplies columns of the normalized rows (bf16 products)
    w = synth.make_norm_weight(D, 5)
    assert torch.equal(codec.kv_a_layernorm(x, w, 0.0), (w.float() * y.float()).to(torch.bfloat16))
