"""Both readers on seeded random shapes against the fp64 oracle at the
north-star tolerance (rtol 2e-2, atol 2e-3): head counts, latent widths,
batch sizes, lengths (tile and page boundaries drawn often), page sizes,
split counts and the reference's window presets (mla_quant/common.py:16)
come from fixed generators, so every run checks the same cases. The fused
writer on random chunked-prefill launches (several requests' chunks at random
offsets in one launch, rows in shuffled slots, a request without ring rows)
against the oracle's writer (mla_fused_writer.py:16-51,110-224): codes within
the +-1 flip budget, params to FP32 rounding, rope and the ring maps exact,
window rows within one bf16 rounding."""
import math

import numpy as np
import pytest
import torch

from tests.helpers import build_pool, make_queries, pool_to_gpu
from tests.test_gpu_decode import ATOL, RTOL, check_against_oracle, run_decode
from tests.test_gpu_extend import run_case
from tests.test_gpu_writer import _compare_layer
from oracle import codec, window
from mla_kv_quant_amd import PackedMLAPool, synth, writer

pytestmark = pytest.mark.gpu

ROPE = {512: 64, 256: 32}
HEADS = [1, 5, 8, 16, 20, 24, 40, 48, 64, 128]
PAGES = [1, 16, 32, 64]
WINDOWS = [(4, 16), (4, 8), (0, 0)]
EDGES = [1, 2, 3, 20, 31, 32, 33, 63, 64, 65, 127, 128, 129]


def _length(g, lo, hi):
    return int(g.choice(EDGES)) if g.random() < 0.4 else int(g.integers(lo, hi))


@pytest.mark.parametrize("seed", range(48))
def test_decode_random_shapes(seed):
    g = np.random.default_rng(1000 + seed)
    D = int(g.choice([512, 256]))
    R, H = ROPE[D], int(g.choice(HEADS))
    B = int(g.integers(1, 6))
    lengths = [_length(g, 1, 1500) for _ in range(B)]
    page = int(g.choice(PAGES))
    P, W = WINDOWS[int(g.integers(0, len(WINDOWS)))]
    splits = [int(g.integers(1, 12)) for _ in range(B)]
    print(f"decode seed {seed}: D={D} H={H} lengths={lengths} page={page} P={P} W={W} splits={splits}", flush=True)
    sm_scale = 1.0 / math.sqrt(192 if D == 512 else 96)
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, page, seed=50 + seed)
    gp = pool_to_gpu(pool)
    q = make_queries(B, H, D, R, sm_scale, seed=70 + seed)
    out, logits, lse = run_decode(gp, q, slots, pages, lengths, reqs, page, splits, 16, P, W, sm_scale)
    check_against_oracle(pool, q, out, lse, slots, lengths, reqs, splits, P, W, sm_scale, D, max_splits=16)


@pytest.mark.parametrize("seed", range(24))
def test_extend_random_shapes(seed):
    g = np.random.default_rng(2000 + seed)
    D = int(g.choice([512, 256]))
    R, H = ROPE[D], int(g.choice(HEADS))
    B = int(g.integers(1, 4))
    prefixes = [0 if g.random() < 0.15 else _length(g, 1, 1200) for _ in range(B)]
    chunks = [_length(g, 1, 150) for _ in range(B)]
    page = int(g.choice(PAGES))
    P, W = WINDOWS[int(g.integers(0, len(WINDOWS)))]
    print(f"extend seed {seed}: D={D} H={H} prefixes={prefixes} chunks={chunks} page={page} P={P} W={W}", flush=True)
    out, ref = run_case(D, R, H, prefixes, chunks, page, seed=90 + seed, P=P, W=W)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.double(), ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("seed", range(16))
def test_writer_random_chunks(seed):
    g = np.random.default_rng(3000 + seed)
    D = int(g.choice([512, 256]))
    R = ROPE[D]
    P, W = WINDOWS[int(g.integers(0, len(WINDOWS)))]
    nreq = int(g.integers(1, 6))
    max_reqs = nreq + 1
    quant = None if g.random() < 0.5 else (float(g.uniform(0.6, 1.2)),)
    if quant is not None:
        quant = (quant[0], codec.signal_gain(quant[0]))
    t, gain = quant if quant is not None else (writer.LM_THRESHOLD, writer.LM_GAIN)
    size = 4096
    rot = synth.make_rotation(D, 500 + seed)
    pool = PackedMLAPool(size, 1, D, R, max_reqs, P, W, device="cuda", rotations=[rot], quantizers=[quant])
    ref = window.new_pool(size + 1, D, R, max_reqs, P, W)
    free = list(g.permutation(np.arange(1, size + 1)))
    loc, pos, seq, req = [], [], [], []
    for b in range(nreq):
        start = 0 if g.random() < 0.4 else _length(g, 1, 600)
        n = _length(g, 1, 300)
        r = b + 1 if b + 1 < max_reqs else max_reqs  # the last request index has no ring rows
        r = max_reqs if g.random() < 0.15 else r
        loc += [int(free.pop()) for _ in range(n)]
        pos += list(range(start, start + n))
        seq += [start + n] * n
        req += [r] * n
    loc, pos, seq, req = (np.array(v, np.int64) for v in (loc, pos, seq, req))
    n = len(loc)
    print(f"writer seed {seed}: D={D} P={P} W={W} rows={n} quant={quant}", flush=True)
    x = synth.make_latent(n, D, 5, seed=7000 + seed)
    pe = synth.make_normal((n, R), 8000 + seed)
    window.write_rows(ref, x, pe, loc, seq, req, rot, t, gain, P, W, max_reqs, positions=pos)
    writer.write_prefill(pool, 0, torch.from_numpy(loc).cuda(), x.cuda(), pe.cuda(), torch.from_numpy(pos).cuda(),
                         torch.from_numpy(seq).cuda(), torch.from_numpy(req).cuda())
    torch.cuda.synchronize()
    _compare_layer(pool, 0, ref, loc, 1e-4)
