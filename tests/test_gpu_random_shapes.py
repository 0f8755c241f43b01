"""Both readers on seeded random shapes against the fp64 oracle at the
north-star tolerance (rtol 2e-2, atol 2e-3): head counts, latent widths,
batch sizes, lengths (tile and page boundaries drawn often), page sizes,
split counts and the reference's window presets (mla_quant/common.py:16)
come from fixed generators, so every run checks the same cases."""
import math

import numpy as np
import pytest
import torch

from tests.helpers import build_pool, make_queries, pool_to_gpu
from tests.test_gpu_decode import ATOL, RTOL, check_against_oracle, run_decode
from tests.test_gpu_extend import run_case

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
