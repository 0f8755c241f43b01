"""GPU parity: extend (chunked prefill) attention over the packed cache against the CPU oracle.

The oracle (``oracle.attention.extend``, SGLang chunk semantics) reads the
prefix rows as the reference's cache holds them -- INT2 rows dequantized and
rounded to bf16, the first P / last W positions of the extended sequence from
the BF16 window -- and attends causally in float64. Tolerance (north star):
rtol 2e-2 / atol 2e-3.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention
from mla_kv_quant_amd import kernels, synth
from tests.helpers import build_pool, index_lists, pool_to_gpu

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 2e-2, 2e-3

CASES = [
    # (name, D, R, H, prefix lengths, chunk lengths, page size)
    ("minicpm3_h40", 256, 32, 40, [300, 0, 1000, 2], [70, 45, 5, 20], 16),
    ("minicpm3_paged32", 256, 32, 40, [513, 64], [130, 1], 32),
    ("dsv2_h16_tokens", 512, 64, 16, [200, 37], [33, 64], 1),
    ("dsv2_h8_paged64", 512, 64, 8, [640, 129], [17, 90], 64),
]


def run_case(D, R, H, prefixes, chunks, page, seed, kc_scale=1.0):
    P, W = 4, 16
    sm = 1.0 / math.sqrt(96 if D == 256 else 192)
    pool, slots, pages, reqs, _ = build_pool(prefixes, D, R, P, W, page, seed=seed)
    gp = pool_to_gpu(pool)
    B = len(prefixes)
    T = sum(chunks)
    sigma = 2.0 / (sm * math.sqrt(D + R))
    q = synth.make_normal((T, H, D + R), seed + 1, std=sigma)
    kc = (kc_scale * torch.cat([synth.make_latent(T, D, 3, seed=seed + 2),
                                synth.make_normal((T, R), seed + 3)], 1)).to(torch.bfloat16)
    qo = np.zeros(B + 1, np.int32)
    qo[1:] = np.cumsum(chunks)
    indptr, indices = index_lists(slots, pages, page)
    out = torch.full((T, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    kernels.extend_fwd(q.to(DEV), kc.to(DEV), torch.from_numpy(qo).to(DEV), indptr, indices,
                       torch.tensor(prefixes, dtype=torch.int64, device=DEV),
                       torch.tensor(reqs, dtype=torch.int64, device=DEV), gp["codes"], gp["params"], gp["rope"],
                       gp["hp"], max(chunks), out, sm, P, W, page)
    torch.cuda.synchronize()
    out = out.float().cpu()
    refs = []
    for b in range(B):
        s, e = qo[b], qo[b + 1]
        ref, _ = attention.extend(pool, q[s:e, :, :D], q[s:e, :, D:], kc[s:e, :D], kc[s:e, D:], slots[b],
                                  prefixes[b], int(reqs[b]), P, W, sm, D, dtype=torch.float64)
        refs.append(ref)
    return out, torch.cat(refs, 0)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_extend_matches_oracle(case):
    name, D, R, H, prefixes, chunks, page = case
    out, ref = run_case(D, R, H, prefixes, chunks, page, seed=7 + len(name))
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.double(), ref, rtol=RTOL, atol=ATOL)


def test_extend_single_token_chunk_equals_decode_semantics():
    """A one-token chunk at position L-1 attends to exactly the decode reader's rows."""
    D, R, H, P, W, page = 256, 32, 40, 4, 16, 16
    L = 700
    out, ref = run_case(D, R, H, [L - 1], [1], page, seed=3)
    torch.testing.assert_close(out.double(), ref, rtol=RTOL, atol=ATOL)


def test_extend_redo_when_scores_outgrow_the_first_tile():
    """The chunk's keys scaled 40x put later scores far above every row's
    first-tile maximum (beyond the kernel's 2^64 headroom), so blocks take the
    second pass with the true maxima; the result must still match."""
    D, R, H, page = 256, 32, 8, 16
    out, ref = run_case(D, R, H, [40, 100], [50, 30], page, seed=11, kc_scale=40.0)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.double(), ref, rtol=RTOL, atol=ATOL)
