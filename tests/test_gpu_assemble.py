"""GPU parity: the dequantize-rows (assemble) kernel against the CPU oracle.

Expected row: the BF16 window row while its slot owns one, else the INT2 row
dequantized and rounded to bf16 (oracle.codec.dequantize); un-rotated rows are
bf16(fp32(row) @ R_eff^T), the cast order of rotate_quantize
(mla_quant/quantizer.py:117-122). Bit-exact in the rotated frame; after the
un-rotation the GEMM's summation order differs from the CPU's, so one bf16
rounding step (2^-8 relative) is allowed.
"""

import numpy as np
import pytest
import torch

from oracle import attention, codec, layout
from mla_kv_quant_amd import PackedMLAPool, kernels
from mla_kv_quant_amd.assemble import assemble_rows
from tests.helpers import bf16_np_to_torch, build_pool, pool_to_gpu

pytestmark = pytest.mark.gpu
DEV = "cuda"


def expected_rows(pool, slots, D):
    codes = layout.unpack_codes(pool["codes"][slots], D)
    prm = torch.from_numpy(pool["params"][slots])
    lat = codec.dequantize(torch.from_numpy(codes), prm[..., 0], prm[..., 1]).to(torch.bfloat16)
    hr = pool["row_of_slot"][slots]
    own = np.zeros(len(slots), bool)
    ok = hr >= 0
    own[ok] = pool["owner_of_row"][hr[ok]] == slots[ok]
    if own.any():
        lat[torch.from_numpy(own)] = bf16_np_to_torch(pool["hp"][hr[own]])
    rope = bf16_np_to_torch(pool["rope"][slots])
    return lat, rope, own


@pytest.mark.parametrize("D,R", [(512, 64), (256, 32)])
def test_assemble_rows_matches_oracle(D, R):
    P, W = 4, 16
    lengths = [300, 17, 90]
    pool, slots, pages, reqs, rot = build_pool(lengths, D, R, P, W, 16, seed=D + 5)
    gp = pool_to_gpu(pool)
    sel = np.concatenate([slots[0][::3], slots[1], slots[2][-40:]])  # window rows included
    lat, rope, own = expected_rows(pool, sel, D)
    assert own.sum() >= 2 * P  # the selection covers window rows
    sl = torch.from_numpy(sel).to(DEV)
    out = torch.full((len(sel), D + R + 8), float("nan"), dtype=torch.bfloat16, device=DEV)
    kernels.assemble_rows(sl, gp["codes"], gp["params"], gp["rope"], gp["hp"], gp["row_of_slot"],
                          gp["owner_of_row"], None, out)
    torch.cuda.synchronize()
    got = out.cpu()
    assert torch.equal(got[:, :D].view(torch.int16), lat.view(torch.int16))
    assert torch.equal(got[:, D:D + R].view(torch.int16), rope.view(torch.int16))
    # un-rotated: bf16(fp32(row) @ R_eff^T)
    r_eff = rot.to(torch.bfloat16)
    out2 = torch.empty(len(sel), D + R, dtype=torch.bfloat16, device=DEV)
    kernels.assemble_rows(sl, gp["codes"], gp["params"], gp["rope"], gp["hp"], gp["row_of_slot"],
                          gp["owner_of_row"], r_eff.to(DEV).contiguous(), out2)
    torch.cuda.synchronize()
    ref = (lat.float() @ r_eff.float().T).to(torch.bfloat16).float()
    torch.testing.assert_close(out2.cpu()[:, :D].float(), ref, rtol=2 ** -7, atol=1e-3)
    assert torch.equal(out2.cpu()[:, D:].view(torch.int16), rope.view(torch.int16))


def test_assemble_rows_restores_rotate_quantize_through_the_pool():
    """Write rows through the pool, read them back un-rotated: INT2 rows equal the
    oracle's rotate_quantize of the original latent (one bf16 step allowed)."""
    from mla_kv_quant_amd import synth, writer
    D, R, P, W, L = 512, 64, 4, 16, 200
    r = synth.make_rotation(D, 77)
    pool = PackedMLAPool(256, 1, D, R, 2, P, W, device=DEV, rotations=[r])
    x = synth.make_latent(L, D, 5, seed=4)
    pe = synth.make_normal((L, R), 5)
    loc = torch.arange(1, L + 1, device=DEV)
    writer.write_prefill(pool, 0, loc, x.to(DEV), pe.to(DEV), torch.arange(L, device=DEV),
                         torch.full((L,), L, device=DEV), torch.ones(L, dtype=torch.int64, device=DEV))
    got = assemble_rows(pool, 0, loc).cpu()
    torch.cuda.synchronize()
    ref = codec.rotate_quantize(x, r)
    # rows whose codes equal the oracle's (a +-1 flip at a rounding boundary of
    # the rotation GEMM moves a whole restored row; such rows are rare)
    ref_codes, _, _, _ = codec.lloyd_codec(codec.rotate(x, r))
    gpu_codes = layout.unpack_codes(pool.c_codes[0].cpu().numpy()[1:L + 1], D)
    same = (gpu_codes == ref_codes.numpy()).all(axis=1)
    same[:P] = same[L - W:] = False  # window rows are returned from their BF16 copies
    assert same.sum() >= 0.95 * (L - P - W)
    torch.testing.assert_close(got[same, :D].float(), ref[same].float(), rtol=2 ** -7, atol=2e-3)
    assert torch.equal(got[:, D:].view(torch.int16), pe.view(torch.int16))
