"""GPU parity: absorbed decode over the packed cache against the CPU oracle.

Tolerance (north star): rtol 2e-2 / atol 2e-3 against the reference's
dequantize-then-attention over its stored rows (``oracle.attention.decode``
"stored64": INT2 rows dequantized in FP32 and rounded to bf16 as
mla_quant/quantizer.py:120 stores them, BF16 window rows, float64 arithmetic),
with no allowance beyond that tolerance. The merged LSE of the split partials
is held to the oracle's LSE within 2e-3.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention, window
from mla_kv_quant_amd import kernels, synth
from mla_kv_quant_amd.decode import packed_mla_decode_gf_fwd, prepare_gf_splits
from tests.helpers import (alloc_slots, build_pool, fused_partials, fused_splits, gpu_pool_to_oracle,
                           gpu_written_pool, index_lists, make_queries, pool_to_gpu)

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
    ("minicpm3_h24", 256, 32, 24, [7, 410], 16, [2, 5]),          # two head groups in one block
    ("minicpm3_h64", 256, 32, 64, [90, 700], 64, [3, 4]),         # two blocks of three and one head groups
    ("dsv2_h32_tp4", 512, 64, 32, [3, 90, 1025], 64, [2, 4, 9]),
    ("dsv2_h8", 512, 64, 8, [48, 777], 16, [3, 6]),
    ("dsv3_h128", 512, 64, 128, [37, 600, 1100], 64, [3, 5, 9]),  # eight head blocks, XCD renumbering
    ("dsv2_h20", 512, 64, 20, [5, 333, 800], 32, [2, 4, 6]),       # a partial second head group
    ("h1", 256, 32, 1, [3, 130, 1000], 1, [1, 2, 5]),               # one head: 15 empty MFMA rows
]
# the reference's window presets (mla_quant/common.py:16): s4r16, s4r8, nowin
WINDOWS = [(4, 16), (4, 8), (0, 0)]


def run_decode(gp, q, slots, pages, lengths, reqs, page, splits, max_splits, P, W, sm_scale, max_reqs=None):
    B, H, DR = q.shape
    D = gp["codes"].shape[1] * 4
    indptr, indices = index_lists(slots, pages, page)
    seq = torch.tensor(lengths, dtype=torch.int64, device=DEV)
    req = torch.tensor(np.asarray(reqs), dtype=torch.int64, device=DEV)
    ns = torch.tensor(splits, dtype=torch.int32, device=DEV)
    logits = torch.full((B, H, max_splits + 1, D), float("nan"), device=DEV)
    lse = torch.full((B, H, max_splits + 1), float("nan"), device=DEV)
    out = torch.empty(B, H, D, dtype=torch.bfloat16, device=DEV)
    kernels.decode_fwd(q.to(DEV), gp["codes"], gp["params"], gp["rope"], gp["hp"], indptr, indices,
                       seq, req, ns, max_splits, logits, lse, out, sm_scale, P, W, page, max_reqs=max_reqs)
    torch.cuda.synchronize()
    logits, lse = fused_partials(logits, lse, B, H, D, max_splits)
    return out.float().cpu(), logits.cpu(), lse.cpu()


def check_against_oracle(pool, q, out, lse, slots, lengths, reqs, splits, P, W, sm_scale, D, max_reqs=None,
                         batch_index=None, max_splits=None):
    """Outputs and merged LSE against the oracle; with ``max_splits`` the
    partials are those of the fused call (split counts capped, no neutral
    window-split partial: its slots 0 .. nq - 1 hold every key)."""
    if max_splits is not None:
        splits = fused_splits(splits, q.shape[1], D, max_splits)
    ref, ref_lse = attention.decode(pool, q[..., :D], q[..., D:], slots, lengths, reqs, P, W, sm_scale, D,
                                    "stored64", max_reqs=max_reqs, batch_index=batch_index)
    idx = list(range(len(lengths))) if batch_index is None else list(batch_index)
    torch.testing.assert_close(out[idx].double(), ref[idx], rtol=RTOL, atol=ATOL)
    for b in idx:
        if lengths[b] == 0:
            continue
        nq = max(splits[b] - 1, 1)
        k = nq if max_splits is not None else nq + 1
        merged = torch.logsumexp(lse[b, :, :k].double(), dim=-1)
        torch.testing.assert_close(merged, ref_lse[b], rtol=0, atol=2e-3)


# every case with s4r16; s4r8 and nowin on the cases that differ in indexing
# (token slots, pages, partial head groups, three head groups per block, XCD renumbering)
ALL_WINDOWS = ("dsv2_token_slots", "dsv2_paged64", "minicpm3_h40", "dsv2_h20", "dsv3_h128", "minicpm3_h64")
PAIRS = [(c, w) for w in WINDOWS for c in CASES if w == (4, 16) or c[0] in ALL_WINDOWS]


@pytest.mark.parametrize("case,win", PAIRS, ids=[f"{c[0]}-P{w[0]}W{w[1]}" for c, w in PAIRS])
def test_decode_matches_oracle(case, win):
    name, D, R, H, lengths, page, splits = case
    P, W = win
    sm_scale = 1.0 / math.sqrt(192 if D == 512 else 96)
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, page, seed=len(name))
    gp = pool_to_gpu(pool)
    q = make_queries(len(lengths), H, D, R, sm_scale, seed=3)
    out, logits, lse = run_decode(gp, q, slots, pages, lengths, reqs, page, splits, 40, P, W, sm_scale)
    check_against_oracle(pool, q, out, lse, slots, lengths, reqs, splits, P, W, sm_scale, D, max_splits=40)
    for b, ns in enumerate(fused_splits(splits, H, D, 40)):
        assert torch.isfinite(logits[b, :, : max(ns - 1, 1)]).all()


def run_partials(gp, q, slots, pages, lengths, reqs, page, splits, max_splits, P, W, sm_scale):
    """Stage 1 at the requested split counts (no cap), then the merge."""
    B, H, DR = q.shape
    D = gp["codes"].shape[1] * 4
    indptr, indices = index_lists(slots, pages, page)
    seq = torch.tensor(lengths, dtype=torch.int64, device=DEV)
    req = torch.tensor(np.asarray(reqs), dtype=torch.int64, device=DEV)
    ns = torch.tensor(splits, dtype=torch.int32, device=DEV)
    logits = torch.full((B, H, max_splits + 1, D), float("nan"), device=DEV)
    lse = torch.full((B, H, max_splits + 1), float("nan"), device=DEV)
    out = torch.empty(B, H, D, dtype=torch.bfloat16, device=DEV)
    kernels.decode_partials(q.to(DEV), gp["codes"], gp["params"], gp["rope"], gp["hp"], indptr, indices, seq, req,
                            ns, max_splits, logits, lse, sm_scale, P, W, page)
    kernels.decode_merge(logits, lse, ns, max_splits, out)
    torch.cuda.synchronize()
    return out.float().cpu(), logits.cpu(), lse.cpu()


def test_split_count_invariance_and_neutral_splits():
    """Every requested split count through the partials entry point (which
    honours it), and the fused call, which caps it, to the same output."""
    D, R, H, P, W = 512, 64, 16, 4, 16
    lengths = [3, 20, 19, 2100, 4097]  # three requests with no INT2 rows at all
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, 64, seed=11)
    gp = pool_to_gpu(pool)
    sm = 1 / math.sqrt(192)
    q = make_queries(len(lengths), H, D, R, sm, seed=5)
    outs = []
    for ns in (1, 2, 3, 8, 33, 129):
        o, logits, lse = run_partials(gp, q, slots, pages, lengths, reqs, 64, [ns] * len(lengths), 129, P, W, sm)
        fused, _, _ = run_decode(gp, q, slots, pages, lengths, reqs, 64, [ns] * len(lengths), 129, P, W, sm)
        torch.testing.assert_close(fused, o, rtol=RTOL, atol=ATOL)
        outs.append(o)
        nq = max(ns - 1, 1)
        # the window rows go with split 0; the window split slot nq is neutral
        assert (lse[:, :, nq] == -1.0e4).all() and (logits[:, :, nq] == 0).all()
        for b in range(3):  # window rows only: every other split is neutral
            assert (lse[b, :, 0] > -1.0e4).all()
            assert (lse[b, :, 1:nq] == -1.0e4).all() and (logits[b, :, 1:nq] == 0).all()
        # more splits than units (window + 32-token tiles): exactly the surplus is neutral
        for b in (3, 4):
            units = 1 + math.ceil((lengths[b] - W) / 32)
            neutral = int((lse[b, 0, :nq] == -1.0e4).sum())
            assert neutral == max(0, nq - units)
            assert ((lse[b, :, :nq] == -1.0e4) == (lse[b, :1, :nq] == -1.0e4)).all()
    for o in outs[1:]:
        # split counts change each wave's reference and so the fp16 rounding
        # of the probabilities: the outputs agree to the attention bar
        torch.testing.assert_close(o, outs[0], rtol=RTOL, atol=ATOL)


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
    ref, _ = attention.decode(pool_np, q[..., :D].cpu(), q[..., D:].cpu(), slots, lengths, reqs, P, W, sm, D,
                              "stored64")
    torch.testing.assert_close(o.double().cpu(), ref, rtol=RTOL, atol=ATOL)
    with pytest.raises(ValueError):
        packed_mla_decode_gf_fwd(q, o, pool, 0, indptr, indices, ns, 8, logits, lse, sm)  # no req indices


def test_partials_then_merge_equals_fused_call():
    """Stage 1 and stage 2 called apart give the fused call's bytes exactly
    (the fused call writes no neutral window-split partial; the separate merge
    gives that partial weight exactly 0)."""
    D, R, H, P, W = 512, 64, 16, 4, 16
    lengths = [5, 300, 1500]
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, 64, seed=31)
    gp = pool_to_gpu(pool)
    sm = 1 / math.sqrt(192)
    q = make_queries(len(lengths), H, D, R, sm, seed=9).to(DEV)
    splits = [2, 5, 9]
    assert fused_splits(splits, H, D, 12) == splits  # three requests: no cap below 12 splits
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
        k = max(n - 1, 1)
        assert torch.equal(l2[b, :, :k].cpu(), logits[b, :, :k])
        assert torch.equal(s2[b, :, :k].cpu(), lse[b, :, :k])
        assert (s2[b, :, k] == -1.0e4).all() and (l2[b, :, k] == 0).all()
    assert torch.equal(o2.float().cpu(), out)


def test_many_sequences_one_block_per_cu():
    """32 requests x 16 splits: 480 working blocks, the first 256 one per CU."""
    D, R, H, P, W = 512, 64, 16, 4, 16
    lengths = [1200 + 53 * i for i in range(32)]
    sm_scale = 1.0 / math.sqrt(192)
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, 64, seed=21)
    gp = pool_to_gpu(pool)
    q = make_queries(len(lengths), H, D, R, sm_scale, seed=22)
    out, logits, lse = run_partials(gp, q, slots, pages, lengths, reqs, 64, [16] * 32, 16, P, W, sm_scale)
    check_against_oracle(pool, q, out, lse, slots, lengths, reqs, [16] * 32, P, W, sm_scale, D)
    assert (lse[:, :, :15] > -1.0e4).all()
    # the fused call caps the split count (one working block per CU): same output
    fused, _, flse = run_decode(gp, q, slots, pages, lengths, reqs, 64, [16] * 32, 16, P, W, sm_scale)
    check_against_oracle(pool, q, fused, flse, slots, lengths, reqs, [16] * 32, P, W, sm_scale, D, max_splits=16)


@pytest.mark.parametrize("page,splits", [(64, 1), (64, 2), (64, 3), (1, 2)], ids=["p64ns1", "p64ns2", "p64ns3", "p1ns2"])
def test_long_context(page, splits):
    """16K-token requests with few splits: up to 128 tiles per wave, every page
    lookup and prefetch slot of the tile ring is exercised."""
    D, R, H, P, W = 512, 64, 16, 4, 16
    lengths = [16384, 16384 - 37] if page == 64 else [9000]
    gp, slots, pages, reqs = gpu_written_pool(lengths, D, R, P, W, page, seed=41 + page)
    sm = 1 / math.sqrt(192)
    q = make_queries(len(lengths), H, D, R, sm, seed=43)
    out, logits, lse = run_decode(gp, q, slots, pages, lengths, reqs, page, [splits] * len(lengths), 4, P, W, sm)
    check_against_oracle(gpu_pool_to_oracle(gp), q, out, lse, slots, lengths, reqs, [splits] * len(lengths), P, W,
                         sm, D, max_splits=4)


@pytest.mark.parametrize("D,R,H", [(512, 64, 16), (256, 32, 40)], ids=["dsv2", "minicpm3"])
def test_128k_context(D, R, H):
    """A 128K-token request beside a 70K one: one split (4097 units, 1025
    tiles for the longest wave) and the reference's 129 requested splits
    (capped by the fused call), against the fp64 oracle."""
    P, W = 4, 16
    lengths = [131072 + 5, 70000]
    gp, slots, pages, reqs = gpu_written_pool(lengths, D, R, P, W, 64, seed=61)
    sm = 1 / math.sqrt(192 if D == 512 else 96)
    q = make_queries(len(lengths), H, D, R, sm, seed=63)
    pool = gpu_pool_to_oracle(gp)
    for splits in ([1, 1], [129, 129]):
        out, logits, lse = run_decode(gp, q, slots, pages, lengths, reqs, 64, splits, 129, P, W, sm)
        check_against_oracle(pool, q, out, lse, slots, lengths, reqs, splits, P, W, sm, D, max_splits=129)


@pytest.mark.parametrize("factor", [100.0, 1000.0])
def test_query_outlier_channels(factor):
    """One query channel per 128-group scaled by 100 or 1000: the products of
    the bf16 query and the stored bf16 rows are exact on the MFMA, so a wide
    dynamic range within a group costs nothing."""
    D, R, H, P, W = 512, 64, 16, 4, 16
    lengths = [700, 2300]
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, 64, seed=51)
    gp = pool_to_gpu(pool)
    sm = 1 / math.sqrt(192)
    q = make_queries(len(lengths), H, D, R, sm, seed=52, logit_std=0.5)
    for g in range(D // 128):
        q[:, :, 128 * g + 17 + 5 * g] *= factor / 50.0
    q[:, :, D + 3] *= factor / 50.0
    q = q.to(torch.bfloat16).float()
    out, logits, lse = run_decode(gp, q.to(torch.bfloat16), slots, pages, lengths, reqs, 64, [3, 5], 8, P, W, sm)
    check_against_oracle(pool, q, out, lse, slots, lengths, reqs, [3, 5], P, W, sm, D, max_splits=8)


def test_request_without_ring_rows_and_reused_index():
    """A request index outside [0, max_reqs) has no ring rows (the writer keeps
    none, mla_fused_writer.py:41), so every position is read from its codes;
    a request index reused by a later request reads the new request's rows."""
    D, R, H, P, W = 512, 64, 16, 4, 16
    max_reqs = 3
    lengths = [500, 300, 260]
    slots, pages, num_slots = alloc_slots(lengths, 64, 61)
    pool = window.new_pool(num_slots, D, R, max_reqs, P, W)
    rot = synth.make_rotation(D, 62)
    # request 2 writes 500 rows, then a new request reuses index 2 with 300 rows;
    # the third request (index 3 = max_reqs) has no ring rows
    reqs = [2, 2, 3]
    for b, L in enumerate(lengths):
        x = synth.make_latent(L, D, 5, seed=63 + b)
        pe = synth.make_normal((L, R), 64 + b)
        window.write_rows(pool, x, pe, slots[b], np.full(L, L), np.full(L, reqs[b]), rot, 0.9810652732849121, 1.16,
                          P, W, max_reqs, positions=np.arange(L))
    assert not (pool["row_of_slot"][slots[2]] >= 0).any()
    gp = pool_to_gpu(pool)
    sm = 1 / math.sqrt(192)
    q = make_queries(3, H, D, R, sm, seed=65)
    sel = [1, 2]  # request 0's ring rows were overwritten by request 1
    out, logits, lse = run_decode(gp, q[sel], [slots[i] for i in sel], [pages[i] for i in sel],
                                  [lengths[i] for i in sel], [reqs[i] for i in sel], 64, [3, 4], 8, P, W, sm,
                                  max_reqs=max_reqs)
    check_against_oracle(pool, q[sel], out, lse, [slots[i] for i in sel], [lengths[i] for i in sel],
                         [reqs[i] for i in sel], [3, 4], P, W, sm, D, max_reqs=max_reqs, max_splits=8)
    with pytest.raises(ValueError):  # hp_c too small for the stated max_reqs
        run_decode(gp, q[sel], [slots[i] for i in sel], [pages[i] for i in sel], [lengths[i] for i in sel],
                   [reqs[i] for i in sel], 64, [3, 4], 8, P, W, sm, max_reqs=max_reqs + 1)


@pytest.mark.parametrize("win", [(4, 16), (0, 0)], ids=["P4W16", "P0W0"])
def test_rescale_when_scores_outgrow_the_reference(win):
    """Logits with std 60 (log2 units ~87): later tiles' maxima exceed each
    wave's reference (its first tile's maximum) by far more than the 2^15 that
    an fp16 probability can hold, so the waves move their references and scale
    their accumulated sums and outputs many times over, in place."""
    D, R, H = 512, 64, 16
    P, W = win
    lengths = [2000, 1300]
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, 64, seed=71)
    gp = pool_to_gpu(pool)
    sm = 1 / math.sqrt(192)
    q = make_queries(len(lengths), H, D, R, sm, seed=72, logit_std=60.0)
    out, logits, lse = run_decode(gp, q, slots, pages, lengths, reqs, 64, [2, 3], 4, P, W, sm)
    assert torch.isfinite(out).all()
    check_against_oracle(pool, q, out, lse, slots, lengths, reqs, [2, 3], P, W, sm, D, max_splits=4)


@pytest.mark.parametrize("D,R,H", [(512, 64, 16), (256, 32, 40)], ids=["dsv2", "minicpm3"])
def test_output_independent_of_page_layout(D, R, H):
    """The same tokens stored in other physical places -- another page size,
    another page shuffle, other request (ring) indices -- are the same values
    in the same order to the kernel, so outputs and LSEs agree bit for bit."""
    P, W = 4, 16
    lengths = [3000, 77, 1, 640]
    n = sum(lengths)
    x = synth.make_latent(n, D, max(1, D // 100), seed=71, device=DEV)
    pe = synth.make_normal((n, R), 72, device=DEV)
    rt = synth.make_rotation(D, 73).to(torch.bfloat16).t().contiguous().to(DEV)
    sm = 1 / math.sqrt(192 if D == 512 else 96)
    q = make_queries(len(lengths), H, D, R, sm, seed=74)
    results = []
    for page, seed, reqs in ((64, 5, [1, 2, 3, 4]), (16, 6, [4, 1, 3, 2]), (1, 7, [2, 4, 1, 3])):
        slots, pages, num_slots = alloc_slots(lengths, page, seed)
        max_reqs = len(lengths) + 1
        hp_rows = 1 + max_reqs * (P + W)
        gp = {"codes": torch.zeros(num_slots, D // 4, dtype=torch.uint8, device=DEV),
              "params": torch.zeros(num_slots, D // 128, 2, dtype=torch.float32, device=DEV),
              "rope": torch.zeros(num_slots, R, dtype=torch.bfloat16, device=DEV),
              "hp": torch.zeros(hp_rows, D, dtype=torch.bfloat16, device=DEV),
              "row_of_slot": torch.full((num_slots,), -1, dtype=torch.int32, device=DEV),
              "owner_of_row": torch.zeros(hp_rows, dtype=torch.int32, device=DEV)}
        loc = torch.from_numpy(np.concatenate(slots)).to(DEV)
        pos = torch.from_numpy(np.concatenate([np.arange(L) for L in lengths])).to(DEV)
        seq = torch.from_numpy(np.concatenate([np.full(L, L) for L in lengths])).to(DEV)
        rq = torch.from_numpy(np.concatenate([np.full(L, r) for L, r in zip(lengths, reqs)])).to(DEV)
        kernels.write_rows(x, pe, rt, loc, seq, pos, rq, gp["codes"], gp["params"], gp["rope"], gp["hp"],
                           gp["row_of_slot"], gp["owner_of_row"], P, W, max_reqs, 0.9810652732849121, 1.16)
        out, logits, lse = run_decode(gp, q, slots, pages, lengths, reqs, page, [5, 2, 1, 3], 8, P, W, sm)
        results.append((out, lse))
    for out, lse in results[1:]:
        assert torch.equal(out, results[0][0])
        assert torch.equal(lse.nan_to_num(0.0), results[0][1].nan_to_num(0.0))
