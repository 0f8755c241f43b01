"""GPU parity: absorbed decode over the packed cache against the CPU oracle.

Tolerance (north star): rtol 2e-2 / atol 2e-3 against the reference's
dequantize-then-attention (``oracle.attention.decode`` "fp32" flavour: cache
rows rounded to bf16 as the reference's QDQ output is, FP32 logits/softmax).
The kernel dequantizes in FP32 without that rounding, so it is also held to
the float64 exact-dequant flavour.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention
from mla_kv_quant_amd import kernels
from mla_kv_quant_amd.decode import packed_mla_decode_gf_fwd, prepare_gf_splits
from tests.helpers import build_pool, index_lists, make_queries, pool_to_gpu

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 2e-2, 2e-3

CASES = [
    # (name, D, R, H, lengths, page_size, splits)
    ("dsv2_token_slots", 512, 64, 16, [1, 4, 5, 20, 21, 22, 37, 100, 333, 1030], 1, [1, 2, 3, 4, 2, 9, 5, 3, 8, 17]),
    ("dsv2_paged64", 512, 64, 16, [64 * 9, 700, 1500, 64, 65, 2049], 64, [4, 4, 8, 2, 3, 32]),
    ("dsv2_paged16", 512, 64, 16, [130, 511, 1000], 16, [3, 5, 9]),
    ("minicpm3_h40", 256, 32, 40, [1, 25, 64, 513, 1200], 32, [2, 3, 4, 6, 9]),
    ("minicpm3_h16", 256, 32, 16, [19, 300, 901], 1, [1, 2, 7]),
    ("dsv2_h32_tp4", 512, 64, 32, [3, 90, 1025], 64, [2, 4, 9]),
    ("dsv2_h8", 512, 64, 8, [48, 777], 16, [3, 6]),
    ("dsv3_h128", 512, 64, 128, [37, 600, 1100], 64, [3, 5, 9]),  # eight head groups, XCD renumbering
    ("dsv2_h20", 512, 64, 20, [5, 333, 800], 32, [2, 4, 6]),       # a partial second head group
    ("h1", 256, 32, 1, [3, 130, 1000], 1, [1, 2, 5]),               # one head: 15 empty MFMA rows
]


def pool_abs_max(pool, D):
    from oracle import codec, layout
    sc = np.abs(pool["params"][..., 0]).max()
    zr = np.abs(pool["params"][..., 1]).max()
    return sc * (3 + zr)


def run_decode(gp, q, slots, pages, lengths, reqs, page, splits, max_splits, P, W, sm_scale):
    B, H, DR = q.shape
    D = gp["codes"].shape[1] * 4
    indptr, indices = index_lists(slots, pages, page)
    seq = torch.tensor(lengths, dtype=torch.int64, device=DEV)
    req = torch.tensor(reqs, dtype=torch.int64, device=DEV)
    ns = torch.tensor(splits, dtype=torch.int32, device=DEV)
    logits = torch.full((B, H, max_splits + 1, D), float("nan"), device=DEV)
    lse = torch.full((B, H, max_splits + 1), float("nan"), device=DEV)
    out = torch.empty(B, H, D, dtype=torch.bfloat16, device=DEV)
    kernels.decode_fwd(q.to(DEV), gp["codes"], gp["params"], gp["rope"], gp["hp"], indptr, indices,
                       seq if page > 1 else seq, req, ns, max_splits, logits, lse, out, sm_scale, P, W, page)
    torch.cuda.synchronize()
    return out.float().cpu(), logits.cpu(), lse.cpu()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_decode_matches_oracle(case):
    name, D, R, H, lengths, page, splits = case
    P, W = 4, 16
    sm_scale = 1.0 / math.sqrt(192 if D == 512 else 96)
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, page, seed=len(name))
    gp = pool_to_gpu(pool)
    q = make_queries(len(lengths), H, D, R, sm_scale, seed=3)
    out, logits, lse = run_decode(gp, q, slots, pages, lengths, reqs, page, splits, 40, P, W, sm_scale)
    ref32, _ = attention.decode(pool, q[..., :D], q[..., D:], slots, lengths, reqs, P, W, sm_scale, D, "fp32")
    ref64, lse64 = attention.decode(pool, q[..., :D], q[..., D:], slots, lengths, reqs, P, W, sm_scale, D, "fp64")
    # primary: the exact (FP32) dequantize-then-attention value
    torch.testing.assert_close(out.double(), ref64, rtol=RTOL, atol=ATOL)
    # secondary: the reference's bf16-stored QDQ rows; the oracle's own storage
    # rounding (<= 2^-9 |c|) is added to the absolute tolerance
    cmax = float(pool_abs_max(pool, D))
    torch.testing.assert_close(out, ref32, rtol=RTOL, atol=ATOL + 2.0 ** -8 * cmax)
    # the merged LSE of the partials equals the exact LSE
    for b, ns in enumerate(splits):
        nq = max(ns - 1, 1)
        l = lse[b, :, : nq + 1].double()
        merged = torch.logsumexp(l, dim=-1)
        torch.testing.assert_close(merged, lse64[b], rtol=0, atol=2e-3)
        assert torch.isfinite(logits[b, :, : nq + 1]).all()


def test_split_count_invariance_and_neutral_splits():
    D, R, H, P, W = 512, 64, 16, 4, 16
    lengths = [0 + 3, 20, 19, 2100, 4097]  # two requests with no INT2 rows at all
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, 64, seed=11)
    gp = pool_to_gpu(pool)
    sm = 1 / math.sqrt(192)
    q = make_queries(len(lengths), H, D, R, sm, seed=5)
    outs = []
    for ns in (1, 2, 3, 8, 33, 129):
        o, logits, lse = run_decode(gp, q, slots, pages, lengths, reqs, 64, [ns] * len(lengths), 129, P, W, sm)
        outs.append(o)
        nq = max(ns - 1, 1)
        # requests 0-2 have no INT2 positions: every quantized split is neutral
        for b in range(3):
            assert (lse[b, :, :nq] == -1.0e4).all() and (logits[b, :, :nq] == 0).all()
        # more splits than tiles: the surplus splits are neutral too
        tiles = math.ceil((lengths[3] - W) / 32)
        if nq > tiles:
            assert (lse[3, :, tiles:nq] == -1.0e4).all()
    for o in outs[1:]:
        # the bf16 output may round differently by one ulp between split counts
        torch.testing.assert_close(o, outs[0], rtol=2 ** -7, atol=1e-3)


def test_packed_mla_decode_entry_and_prepare_splits():
    from mla_kv_quant_amd import PackedMLAPool
    D, R, H, P, W = 512, 64, 16, 4, 16
    lengths = [50, 600]
    pool_np, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, 1, seed=21, max_reqs=4)
    gp = pool_to_gpu(pool_np)
    pool = PackedMLAPool(pool_np["codes"].shape[0] - 1, 1, D, R, 4, P, W, device=DEV)
    pool.c_codes[0].copy_(gp["codes"]), pool.c_params[0].copy_(gp["params"])
    pool.rope_buf[0].copy_(gp["rope"]), pool.hp_c[0].copy_(gp["hp"])
    sm = 1 / math.sqrt(192)
    q = make_queries(2, H, D, R, sm, seed=8).to(DEV)
    indptr, indices = index_lists(slots, pages, 1)
    ns = torch.tensor([3, 1], dtype=torch.int32, device=DEV)
    quant, merge = torch.empty_like(ns), torch.empty_like(ns)
    prepare_gf_splits(ns, quant, merge)
    torch.cuda.synchronize()
    assert quant.tolist() == [2, 1] and merge.tolist() == [3, 2]
    o = torch.empty(2, H, D, dtype=torch.bfloat16, device=DEV)
    logits = torch.empty(4, H, 9, D, device=DEV)
    lse = torch.empty(4, H, 9, device=DEV)
    packed_mla_decode_gf_fwd(q, o, pool, 0, indptr, indices, ns, 8, logits, lse, sm,
                             seq_lens=torch.tensor(lengths, device=DEV),
                             req_pool_indices=torch.tensor(reqs, device=DEV))
    ref, _ = attention.decode(pool_np, q[..., :D].cpu(), q[..., D:].cpu(), slots, lengths, reqs, P, W, sm, D, "fp64")
    torch.testing.assert_close(o.double().cpu(), ref, rtol=RTOL, atol=ATOL)
    with pytest.raises(ValueError):
        packed_mla_decode_gf_fwd(q, o, pool, 0, indptr, indices, ns, 8, logits, lse, sm)  # no req indices


def test_partials_then_merge_equals_fused_call():
    """Stage 1 and stage 2 called apart give the fused call's bytes exactly."""
    D, R, H, P, W = 512, 64, 16, 4, 16
    lengths = [5, 300, 1500]
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, 64, seed=31)
    gp = pool_to_gpu(pool)
    sm = 1 / math.sqrt(192)
    q = make_queries(len(lengths), H, D, R, sm, seed=9).to(DEV)
    splits = [2, 5, 9]
    out, logits, lse = run_decode(gp, q, slots, pages, lengths, reqs, 64, splits, 12, P, W, sm)
    indptr, indices = index_lists(slots, pages, 64)
    seq = torch.tensor(lengths, dtype=torch.int64, device=DEV)
    req = torch.tensor(reqs, dtype=torch.int64, device=DEV)
    ns = torch.tensor(splits, dtype=torch.int32, device=DEV)
    B = len(lengths)
    l2 = torch.full((B, H, 13, D), float("nan"), device=DEV)
    s2 = torch.full((B, H, 13), float("nan"), device=DEV)
    o2 = torch.empty(B, H, D, dtype=torch.bfloat16, device=DEV)
    kernels.decode_partials(q, gp["codes"], gp["params"], gp["rope"], gp["hp"], indptr, indices, seq, req, ns, 12,
                            l2, s2, sm, P, W, 64)
    kernels.decode_merge(l2, s2, ns, 12, o2)
    torch.cuda.synchronize()
    for b, n in enumerate(splits):
        k = max(n - 1, 1) + 1
        assert torch.equal(l2[b, :, :k].cpu(), logits[b, :, :k])
        assert torch.equal(s2[b, :, :k].cpu(), lse[b, :, :k])
    assert torch.equal(o2.float().cpu(), out)


def test_first_round_tile_shares():
    """32 requests x 16 splits with max_kv_splits 16: every block is resident
    (two per CU on the 256-CU MI355X), so the first dispatch round's splits get
    the larger tile shares. Same oracle bars as the other cases, and the merged
    LSE over all partials equals the exact one."""
    D, R, H, P, W = 512, 64, 16, 4, 16
    lengths = [1200 + 53 * i for i in range(32)]
    sm_scale = 1.0 / math.sqrt(192)
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, 64, seed=21)
    gp = pool_to_gpu(pool)
    q = make_queries(len(lengths), H, D, R, sm_scale, seed=22)
    out, logits, lse = run_decode(gp, q, slots, pages, lengths, reqs, 64, [16] * 32, 16, P, W, sm_scale)
    ref64, lse64 = attention.decode(pool, q[..., :D], q[..., D:], slots, lengths, reqs, P, W, sm_scale, D, "fp64")
    torch.testing.assert_close(out.double(), ref64, rtol=RTOL, atol=ATOL)
    merged = torch.logsumexp(lse[:, :, :16].double(), dim=-1)
    torch.testing.assert_close(merged, lse64, rtol=0, atol=2e-3)
    # the first-round splits (0..7 here) hold more tiles than the others: their
    # partials are non-neutral, and so are those of the rest
    assert (lse[:, :, :15] > -1.0e4).all()
