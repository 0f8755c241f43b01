"""GPU parity: kv_a_layernorm fused in front of the cache writer.

The fused launch must store exactly what the plain writer stores for the rows
it normalized (same MFMA operands, same order: bit-identical cache), and its
normalized rows must match ``oracle.codec.kv_a_layernorm`` (pinned against
transformers' DeepseekV2RMSNorm in ``tests/test_oracle_norm.py``). The FP32
sum of squares runs in another order than torch's, so a row's inverse RMS may
differ in its last bit and move the first rounding, ``bf16(x * r)``, by one
unit on a small fraction of the elements; the weight multiplies that unit into
at most two units of the result (one unit of ``h`` at the bottom of its binade
is 2^-7 of ``h``, one unit of ``w * h`` at the top of its binade is 2^-8). The whole chain against the oracle then holds the
writer's code-flip budget.
"""

import numpy as np
import pytest
import torch

from oracle import codec, window
from mla_kv_quant_amd import PackedMLAPool, synth, writer
from tests.test_gpu_writer import _compare_layer

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS = 1e-6


def _norm_close(y: torch.Tensor, ref: torch.Tensor, budget: float):
    """bf16 ``y`` equals ``ref`` except for <= budget of the elements, each at most two bf16 units away."""
    yi, ri = y.cpu().view(torch.int16).int(), ref.view(torch.int16).int()
    diff = (yi - ri).abs()
    nbad = int((diff != 0).sum())
    assert int(diff.max()) <= 2, "a normalized element differs by more than two bf16 units"
    assert nbad <= budget * y.numel(), f"{nbad} of {y.numel()} normalized elements differ"
    return nbad


def _pools(D, R, size, rots, quant, max_reqs=6, P=4, W=16):
    return [PackedMLAPool(size, len(rots), D, R, max_reqs, P, W, device=DEV, rotations=rots, quantizers=quant)
            for _ in range(2)]


def _same_layer(a: PackedMLAPool, b: PackedMLAPool, li: int):
    for name in ("c_codes", "c_params", "rope_buf", "hp_c"):
        x, y = getattr(a, name)[li], getattr(b, name)[li]
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), name
    assert torch.equal(a.hp_row_of_slot, b.hp_row_of_slot)
    assert torch.equal(a.hp_owner_of_row, b.hp_owner_of_row)


@pytest.mark.parametrize("D,R", [(512, 64), (256, 32)])
def test_norm_prefill_matches_writer_and_oracle(D, R):
    n, size = 3001, 4096
    rots = [synth.make_rotation(D, 300), None]
    quant = [(0.8, codec.signal_gain(0.8)), None]
    a, b = _pools(D, R, size, rots, quant)
    w = synth.make_norm_weight(D, 21)
    kv_a = synth.make_kv_a(n, D, 22)
    kv_a[5] = 0.0                                     # zero row: eps keeps it finite
    pe = synth.make_normal((n, R), 23)
    rng = np.random.default_rng(2)
    loc = rng.permutation(np.arange(1, size + 1))[:n].astype(np.int64)
    lens = [1, 40, 960, 2000]                         # four requests, positions 0..L-1
    pos = np.concatenate([np.arange(L) for L in lens])
    seq = np.concatenate([np.full(L, L) for L in lens])
    req = np.concatenate([np.full(L, i + 1) for i, L in enumerate(lens)])
    dev = lambda v: torch.from_numpy(v).to(DEV)
    ref_y = codec.kv_a_layernorm(kv_a, w, EPS)
    for li in range(2):
        y = torch.empty(n, D, dtype=torch.bfloat16, device=DEV)
        writer.norm_write_prefill(a, li, dev(loc), kv_a.to(DEV), pe.to(DEV), dev(pos), dev(seq), dev(req), w.to(DEV),
                                  EPS, latent_out=y)
        torch.cuda.synchronize()
        assert torch.equal(y[5].cpu(), torch.zeros(D, dtype=torch.bfloat16))
        _norm_close(y, ref_y, 1e-4)
        # the plain writer on the kernel's own normalized rows: bit-identical cache
        # (for the rotated layer; an un-rotated layer's plain writer packs the rows
        # directly, summing in another order, and meets the oracle check below)
        writer.write_prefill(b, li, dev(loc), y, pe.to(DEV), dev(pos), dev(seq), dev(req))
        torch.cuda.synchronize()
        if rots[li] is not None:
            _same_layer(a, b, li)
        # the cache against the oracle writer on the normalized rows (the GPU's,
        # which equal the oracle's but for the rare last-bit cases counted above)
        t, g = quant[li] if quant[li] else (writer.LM_THRESHOLD, writer.LM_GAIN)
        ref = window.new_pool(size + 1, D, R, 6, 4, 16)
        window.write_rows(ref, y.cpu(), pe, loc, seq, req, rots[li], t, g, 4, 16, 6, positions=pos)
        _compare_layer(a, li, ref, loc, 1e-4)


@pytest.mark.parametrize("D,R", [(512, 64), (256, 32)])
def test_norm_writer_many_tiles_per_wave(D, R):
    """Enough rows that every wave runs several tiles (the next tile's first
    K-steps are loaded during the current one); no latent_out."""
    n = 80_000 + 37
    size = n + 16
    rots = [synth.make_rotation(D, 301)]
    a, b = _pools(D, R, size, rots, [None], max_reqs=2, P=2, W=4)
    w = synth.make_norm_weight(D, 31).to(DEV)
    kv_a = synth.make_kv_a(n, D, 32, device=DEV)
    pe = synth.make_normal((n, R), 33, device=DEV)
    loc = torch.arange(1, n + 1, device=DEV)
    pos = torch.arange(n, device=DEV)
    seq = torch.full((n,), n, device=DEV)
    req = torch.ones(n, dtype=torch.int64, device=DEV)
    writer.norm_write_prefill(a, 0, loc, kv_a, pe, pos, seq, req, w, EPS)
    y = codec.kv_a_layernorm(kv_a.cpu(), w.cpu(), EPS)
    # rows whose GPU normalization differs from the oracle's go through the plain
    # writer with the GPU's rows; compare the caches bit for bit elsewhere
    writer.write_prefill(b, 0, loc, y.to(DEV), pe, pos, seq, req)
    torch.cuda.synchronize()
    ya = torch.empty(n, D, dtype=torch.bfloat16, device=DEV)
    a2, _ = _pools(D, R, size, rots, [None], max_reqs=2, P=2, W=4)
    writer.norm_write_prefill(a2, 0, loc, kv_a, pe, pos, seq, req, w, EPS, latent_out=ya)
    torch.cuda.synchronize()
    _norm_close(ya, y, 1e-4)
    same = (ya.cpu().view(torch.int16) == y.view(torch.int16)).all(-1).to(DEV)
    assert int(same.sum()) >= n - max(2, int(1e-4 * n * D))
    rows = loc[same]
    for name in ("c_codes", "c_params", "rope_buf"):
        x1, x2 = getattr(a, name)[0][rows], getattr(b, name)[0][rows]
        assert torch.equal(x1.view(torch.uint8), x2.view(torch.uint8)), name
    assert torch.equal(a.c_codes[0], a2.c_codes[0]) and torch.equal(a.hp_c[0], a2.hp_c[0])
    assert torch.equal(a.hp_row_of_slot, b.hp_row_of_slot) and torch.equal(a.hp_owner_of_row, b.hp_owner_of_row)


def test_norm_decode_store_gatekeeping_and_parity():
    D, R, P, W = 512, 64, 4, 16
    rots = [synth.make_rotation(D, 302), None]
    a, b = _pools(D, R, 64, rots, [None, None], max_reqs=4, P=P, W=W)
    w = synth.make_norm_weight(D, 41).to(DEV)
    kv_a = synth.make_kv_a(4, D, 42, device=DEV)
    pe = synth.make_normal((4, R), 43, device=DEV)
    seq = torch.tensor([5, 30, 2, 1], device=DEV)
    req = torch.tensor([1, 2, 3, 0], device=DEV)
    loc = torch.tensor([7, 8, 9, 0], device=DEV)           # slot 0: graph padding
    for pool in (a, b):
        pool.set_window_meta(False, seq, req)
    assert not writer.try_fast_norm_decode_store(a, 0, loc, kv_a, pe, w, EPS)   # not a decode step
    for pool in (a, b):
        pool.set_window_meta(True, seq, req)
    for li in range(2):
        y = torch.empty(4, D, dtype=torch.bfloat16, device=DEV)
        assert writer.try_fast_norm_decode_store(a, li, loc, kv_a, pe, w, EPS, latent_out=y)
        assert writer.try_fast_decode_store(b, li, loc, y, pe)
        torch.cuda.synchronize()
        _norm_close(y, codec.kv_a_layernorm(kv_a.cpu(), w.cpu(), EPS), 1e-3)
        if li == 0:
            _same_layer(a, b, li)
        else:
            # un-rotated layer: the fused path rotates by the identity (exact products),
            # the plain one packs the rows directly with its own summation order; both
            # against the oracle writer on the GPU's normalized rows
            ref = window.new_pool(65, D, R, 4, P, W)
            window.write_rows(ref, y.cpu(), pe.cpu(), loc.cpu().numpy(), seq.cpu().numpy(), req.cpu().numpy(), None,
                              writer.LM_THRESHOLD, writer.LM_GAIN, P, W, 4)
            _compare_layer(a, li, ref, np.array([7, 8, 9]), 1e-5)
            _compare_layer(b, li, ref, np.array([7, 8, 9]), 1e-5)
    with pytest.raises(ValueError):
        writer.try_fast_norm_decode_store(a, 0, loc, kv_a, pe, w[:256].contiguous(), EPS)
    with pytest.raises(ValueError):
        writer.try_fast_norm_decode_store(a, 0, loc, kv_a, pe, w, float("nan"))
