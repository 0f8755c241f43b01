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


def run_case(D, R, H, prefixes, chunks, page, seed, kc_scale=1.0, P=4, W=16, max_reqs=None, reqs=None):
    sm = 1.0 / math.sqrt(96 if D == 256 else 192)
    pool, slots, pages, breqs, _ = build_pool(prefixes, D, R, P, W, page, seed=seed, max_reqs=max_reqs)
    reqs = breqs if reqs is None else np.asarray(reqs)
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
                       gp["hp"], max(chunks), out, sm, P, W, page, max_reqs=max_reqs)
    torch.cuda.synchronize()
    out = out.float().cpu()
    refs = []
    for b in range(B):
        s, e = qo[b], qo[b + 1]
        ref, _ = attention.extend(pool, q[s:e, :, :D], q[s:e, :, D:], kc[s:e, :D], kc[s:e, D:], slots[b],
                                  prefixes[b], int(reqs[b]), P, W, sm, D, dtype=torch.float64, max_reqs=max_reqs)
        refs.append(ref)
    return out, torch.cat(refs, 0)


WINDOWS = [(4, 16), (4, 8), (0, 0)]  # s4r16, s4r8, nowin (mla_quant/common.py:16)


@pytest.mark.parametrize("win", WINDOWS, ids=[f"P{p}W{w}" for p, w in WINDOWS])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_extend_matches_oracle(case, win):
    name, D, R, H, prefixes, chunks, page = case
    if win != (4, 16) and name not in ("minicpm3_h40", "dsv2_h16_tokens"):
        pytest.skip("other window presets run on a representative subset")
    out, ref = run_case(D, R, H, prefixes, chunks, page, seed=7 + len(name), P=win[0], W=win[1])
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.double(), ref, rtol=RTOL, atol=ATOL)


def test_extend_request_without_ring_rows():
    """A request index outside [0, max_reqs) reads its whole prefix from the codes."""
    D, R, H, page = 256, 32, 16, 16
    out, ref = run_case(D, R, H, [300, 120], [20, 9], page, seed=5, max_reqs=3, reqs=[1, 3])
    torch.testing.assert_close(out.double(), ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("D,R,H", [(256, 32, 40), (512, 64, 16)])
def test_extend_single_token_chunk_equals_decode(D, R, H):
    """A one-token chunk at position L-1 whose key is the cache's stored row of
    that position attends to exactly the rows the decode reader sees at length
    L: both readers agree to one bf16 ulp of the output (2^-7 relative at
    most: their FP32 results, which differ in accumulation order only, may
    round to neighbouring bf16 values) plus atol 1e-3."""
    P, W, page, L = 4, 16, 16, 700
    sm = 1.0 / math.sqrt(96 if D == 256 else 192)
    pool, slots, pages, reqs, _ = build_pool([L], D, R, P, W, page, seed=3)
    gp = pool_to_gpu(pool)
    q = synth.make_normal((1, H, D + R), 4, std=2.0 / (sm * math.sqrt(D + R)))
    # decode at length L
    indptr, indices = index_lists(slots, pages, page)
    logits = torch.empty(1, H, 5, D, device=DEV)
    lse = torch.empty(1, H, 5, device=DEV)
    od = torch.empty(1, H, D, dtype=torch.bfloat16, device=DEV)
    kernels.decode_fwd(q.to(DEV), gp["codes"], gp["params"], gp["rope"], gp["hp"], indptr, indices,
                       torch.tensor([L], device=DEV), torch.tensor(reqs, dtype=torch.int64, device=DEV),
                       torch.tensor([3], dtype=torch.int32, device=DEV), 4, logits, lse, od, sm, P, W, page)
    # extend: prefix L-1, the chunk's key = the stored window row of position L-1 and its rope
    from oracle import window as owin
    ring = int(owin.ring_row(int(reqs[0]), L - 1, P, W))
    kc = torch.cat([gp["hp"][ring], gp["rope"][int(slots[0][L - 1])]])[None]
    oe = torch.empty(1, H, D, dtype=torch.bfloat16, device=DEV)
    kernels.extend_fwd(q.to(DEV), kc.contiguous(), torch.tensor([0, 1], dtype=torch.int32, device=DEV), indptr,
                       indices, torch.tensor([L - 1], device=DEV), torch.tensor(reqs, dtype=torch.int64, device=DEV),
                       gp["codes"], gp["params"], gp["rope"], gp["hp"], 1, oe, sm, P, W, page)
    torch.cuda.synchronize()
    torch.testing.assert_close(oe.float().cpu(), od.float().cpu(), rtol=2 ** -7, atol=1e-3)
    ref, _ = attention.decode(pool, q[..., :D].float(), q[..., D:].float(), slots, [L], reqs, P, W, sm, D,
                              "stored64")
    torch.testing.assert_close(oe.float().cpu().double(), ref, rtol=RTOL, atol=ATOL)


def test_extend_redo_when_scores_outgrow_the_first_tile():
    """The chunk's keys scaled 40x put later scores far above every row's
    first-tile maximum (beyond the kernel's 2^64 headroom), so blocks take the
    second pass with the true maxima; the result must still match."""
    D, R, H, page = 256, 32, 8, 16
    out, ref = run_case(D, R, H, [40, 100], [50, 30], page, seed=11, kc_scale=40.0)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.double(), ref, rtol=RTOL, atol=ATOL)
