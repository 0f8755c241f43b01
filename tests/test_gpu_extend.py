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
from tests.helpers import build_pool, index_lists, pool_to_gpu, rotated_latent

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 2e-2, 2e-3

CASES = [
    # (name, D, R, H, prefix lengths, chunk lengths, page size)
    ("minicpm3_h40", 256, 32, 40, [300, 0, 1000, 2], [70, 45, 5, 20], 16),
    ("minicpm3_paged32", 256, 32, 40, [513, 64], [130, 1], 32),
    ("dsv2_h16_tokens", 512, 64, 16, [200, 37], [33, 64], 1),
    ("dsv2_h8_paged64", 512, 64, 8, [640, 129], [17, 90], 64),
    ("dsv3_h128", 512, 64, 128, [300, 40], [20, 7], 64),        # eight head blocks
    ("minicpm3_h64", 256, 32, 64, [90, 700], [12, 33], 64),
]


def run_case(D, R, H, prefixes, chunks, page, seed, rope_scale=1.0, P=4, W=16, max_reqs=None, reqs=None,
             rotated_keys=True, flavour="fp"):
    """Extend over a pool written with a seeded rotation. The chunk's keys are
    latent rows in that rotated frame, as the reader receives them (the cache
    rows and the chunk rows are the same rotated latent); ``rotated_keys=False``
    takes the synthetic rows with their x20 outlier channels as they are."""
    sm = 1.0 / math.sqrt(96 if D == 256 else 192)
    pool, slots, pages, breqs, rot = build_pool(prefixes, D, R, P, W, page, seed=seed, max_reqs=max_reqs)
    reqs = breqs if reqs is None else np.asarray(reqs)
    gp = pool_to_gpu(pool)
    B = len(prefixes)
    T = sum(chunks)
    sigma = 2.0 / (sm * math.sqrt(D + R))
    q = synth.make_normal((T, H, D + R), seed + 1, std=sigma)
    lat = rotated_latent(T, D, 3, seed + 2, rot) if rotated_keys else synth.make_latent(T, D, 3, seed=seed + 2)
    kc = torch.cat([lat.float(), rope_scale * synth.make_normal((T, R), seed + 3).float()], 1).to(torch.bfloat16)
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
                                  prefixes[b], int(reqs[b]), P, W, sm, D, dtype=torch.float64, max_reqs=max_reqs,
                                  flavour=flavour)
        refs.append(ref)
    return out, torch.cat(refs, 0)


WINDOWS = [(4, 16), (4, 8), (0, 0)]  # s4r16, s4r8, nowin (mla_quant/common.py:16)


# every case with s4r16; s4r8 and nowin on token slots, a partial head group and many head blocks
ALL_WINDOWS = ("minicpm3_h40", "dsv2_h16_tokens", "dsv3_h128", "minicpm3_h64")
PAIRS = [(c, w) for w in WINDOWS for c in CASES if w == (4, 16) or c[0] in ALL_WINDOWS]


@pytest.mark.parametrize("case,win", PAIRS, ids=[f"{c[0]}-P{w[0]}W{w[1]}" for c, w in PAIRS])
def test_extend_matches_oracle(case, win):
    name, D, R, H, prefixes, chunks, page = case
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
    L: both readers agree to the attention bar (they round their fp16
    probabilities against different references, so not bit for bit)."""
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
    torch.testing.assert_close(oe.float().cpu(), od.float().cpu(), rtol=RTOL, atol=ATOL)
    ref, _ = attention.decode(pool, q[..., :D].float(), q[..., D:].float(), slots, [L], reqs, P, W, sm, D,
                              "stored64")
    torch.testing.assert_close(oe.float().cpu().double(), ref, rtol=RTOL, atol=ATOL)


def test_extend_rescale_when_scores_outgrow_the_reference():
    """The chunk's rope keys scaled 40x put later scores far above every row's
    first-tile reference (beyond the 2^15 an fp16 probability holds), so the
    rows move their references and scale their sums and outputs in place,
    many times over; the result must still match. (The values attended over,
    the latent rows, keep their size: large values are the subject of
    test_extend_unrotated_outlier_keys_no_worse_than_the_reference.)"""
    D, R, H, page = 256, 32, 8, 16
    out, ref = run_case(D, R, H, [40, 100], [50, 30], page, seed=11, rope_scale=40.0)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.double(), ref, rtol=RTOL, atol=ATOL)


def test_extend_unrotated_outlier_keys_no_worse_than_the_reference():
    """Chunk keys taken un-rotated, with x20 outlier channels (|v| up to ~60),
    where outputs cancel between keys of nearly equal weight: the fp16
    probabilities leave up to 2^-12 |v_i - v_j| there, above the 2e-3 bar
    against float64 at single elements. The reference's own dequantize-then-
    BF16 attention (transformers' eager path, bf16 probabilities) is further
    from float64 on the same data: the kernel's largest and RMS errors
    against float64 must not exceed the reference's, and all but 1e-4 of the
    elements stay within the bar."""
    D, R, H, page = 256, 32, 40, 16
    prefixes, chunks = [300, 0, 1000, 2], [70, 45, 5, 20]
    out, ref = run_case(D, R, H, prefixes, chunks, page, seed=19, rotated_keys=False)
    _, eager = run_case(D, R, H, prefixes, chunks, page, seed=19, rotated_keys=False, flavour="bf16_eager")
    assert torch.isfinite(out).all()
    err, err_ref = (out.double() - ref).abs(), (eager.double() - ref).abs()
    assert err.max() <= err_ref.max()
    assert err.pow(2).mean().sqrt() <= err_ref.pow(2).mean().sqrt()
    outside = (err > ATOL + RTOL * ref.abs()).double().mean().item()
    print(f"max|err| {err.max():.2e} (reference bf16: {err_ref.max():.2e}), beyond the bar: {outside:.2e}")
    assert outside <= 1e-4


def test_extend_rotated_keys_cancellation_tail():
    """A case from a wider seeded sweep (128 heads, rotated keys, s4r8): one
    output element of 6.3 M, of magnitude 0.007 where its keys' values cancel,
    lands 2.6e-3 from float64 against a bar of 2.15e-3 -- the fp16
    probabilities' 2^-12 relative rounding times |v|. The reference's BF16
    eager attention misses the bar on about 12 % of this case's elements:
    the kernel's largest and RMS errors stay at or below the reference's,
    every element stays within twice the bar, and at most 1e-6 of the
    elements pass the bar itself."""
    D, R, H, page = 256, 32, 128, 32
    prefixes, chunks = [1020, 31, 300], [47, 71, 74]
    out, ref = run_case(D, R, H, prefixes, chunks, page, seed=217, P=4, W=8)
    _, eager = run_case(D, R, H, prefixes, chunks, page, seed=217, P=4, W=8, flavour="bf16_eager")
    assert torch.isfinite(out).all()
    err, err_ref = (out.double() - ref).abs(), (eager.double() - ref).abs()
    bar = ATOL + RTOL * ref.abs()
    assert err.max() <= err_ref.max()
    assert err.pow(2).mean().sqrt() <= err_ref.pow(2).mean().sqrt()
    assert (err <= 2 * bar).all()
    outside = (err > bar).double().mean().item()
    print(f"max|err| {err.max():.2e} (reference bf16: {err_ref.max():.2e}), beyond the bar: {outside:.2e}")
    assert outside <= 1e-6


def test_extend_short_workspace():
    """A workspace shorter than the key rows the caller states is rejected
    before any launch (ValueError, output untouched); a caller that states too
    few key rows gets NaN outputs for the sequences that do not fit, never
    silently wrong ones."""
    D, R, H, page, P, W = 256, 32, 8, 16, 4, 16
    prefixes, chunks = [300, 200], [40, 30]
    sm = 1.0 / math.sqrt(96)
    pool, slots, pages, reqs, _ = build_pool(prefixes, D, R, P, W, page, seed=13)
    gp = pool_to_gpu(pool)
    T = sum(chunks)
    q = synth.make_normal((T, H, D + R), 14, std=2.0 / (sm * math.sqrt(D + R))).to(DEV)
    kc = torch.cat([synth.make_latent(T, D, 3, seed=15), synth.make_normal((T, R), 16)], 1).to(DEV)
    qo = torch.tensor([0, chunks[0], T], dtype=torch.int32, device=DEV)
    indptr, indices = index_lists(slots, pages, page)
    args = (q, kc, qo, indptr, indices, torch.tensor(prefixes, dtype=torch.int64, device=DEV),
            torch.tensor(reqs, dtype=torch.int64, device=DEV), gp["codes"], gp["params"], gp["rope"], gp["hp"],
            max(chunks))
    rows = sum(prefixes) + T
    out = torch.zeros(T, H, D, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(rows - 1, D + R, dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError, match="short"):
        kernels.extend_fwd(*args, out, sm, P, W, page, workspace=ws, key_rows=rows)
    with pytest.raises(ValueError, match="short"):
        kernels.extend_fwd(*args, out, sm, P, W, page, workspace=ws)  # key rows read back from the device
    torch.cuda.synchronize()
    assert (out == 0).all()
    # stated one row short: the second sequence (rows 340 .. 569) does not fit
    kernels.extend_fwd(*args, out, sm, P, W, page, workspace=ws, key_rows=rows - 1)
    torch.cuda.synchronize()
    got = out.float().cpu()
    assert torch.isnan(got[chunks[0]:]).all()
    ws_ok = torch.empty(rows, D + R, dtype=torch.float16, device=DEV)
    ok = torch.empty_like(out)
    kernels.extend_fwd(*args, ok, sm, P, W, page, workspace=ws_ok, key_rows=rows)
    torch.cuda.synchronize()
    assert torch.equal(got[:chunks[0]], ok.float().cpu()[:chunks[0]])  # the first sequence fits: same output
    assert torch.isfinite(ok.float()).all()


def test_extend_hf_chunk_semantics():
    """HF cache semantics (mla_quant/cache.py:1028-1039): the chunk is written
    into the cache before attention, so its rows outside the extended
    sequence's window enter as their Lloyd QDQ rounded to bf16 and its window
    rows as BF16. With the whole extended sequences in the cache (written by
    the oracle's writer), the dequantize-rows kernel reads the chunk's stored
    rows back, in the rotated frame, bit for bit equal to the oracle's
    chunk_rows(..., "qdq") of the chunk's FP32 rotated latent; fed to the
    extend reader as the chunk's keys they give the output of
    oracle.attention.extend(chunk_mode="qdq") at the attention bar."""
    from oracle import codec

    D, R, H, page, P, W = 256, 32, 16, 16, 4, 16
    prefixes, chunks = [200, 37], [40, 9]  # the second chunk is shorter than W: prefix rows stay in the window
    lengths = [p + c for p, c in zip(prefixes, chunks)]
    sm = 1.0 / math.sqrt(96)
    seed = 23
    pool, slots, pages, reqs, rot = build_pool(lengths, D, R, P, W, page, seed=seed)
    gp = pool_to_gpu(pool)
    B, T = len(prefixes), sum(chunks)
    chunk_slots = np.concatenate([slots[b][prefixes[b]:lengths[b]] for b in range(B)]).astype(np.int64)
    kc = torch.empty(T, D + R, dtype=torch.bfloat16, device=DEV)
    kernels.assemble_rows(torch.from_numpy(chunk_slots).to(DEV), gp["codes"], gp["params"], gp["rope"], gp["hp"],
                          gp["row_of_slot"], gp["owner_of_row"], None, kc)
    q = synth.make_normal((T, H, D + R), seed + 1, std=2.0 / (sm * math.sqrt(D + R)))
    qo = np.zeros(B + 1, np.int32)
    qo[1:] = np.cumsum(chunks)
    indptr, indices = index_lists([s[:p] for s, p in zip(slots, prefixes)], pages, page)
    out = torch.full((T, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    kernels.extend_fwd(q.to(DEV), kc, torch.from_numpy(qo).to(DEV), indptr, indices,
                       torch.tensor(prefixes, dtype=torch.int64, device=DEV),
                       torch.tensor(reqs, dtype=torch.int64, device=DEV), gp["codes"], gp["params"], gp["rope"],
                       gp["hp"], max(chunks), out, sm, P, W, page)
    torch.cuda.synchronize()
    kc, out = kc.float().cpu(), out.float().cpu()
    for b in range(B):
        s, e, L, pf = qo[b], qo[b + 1], lengths[b], prefixes[b]
        x = synth.make_latent(L, D, max(1, D // 100), seed=seed * 31 + b)  # the rows build_pool wrote
        pe = synth.make_normal((L, R), seed * 37 + b)
        lat32 = codec.rotate(x, rot)[pf:L]
        assert torch.equal(kc[s:e, :D], attention.chunk_rows(lat32, pf, P, W, "qdq"))
        assert torch.equal(kc[s:e, D:], pe[pf:L].float())
        ref, _ = attention.extend(pool, q[s:e, :, :D], q[s:e, :, D:], lat32, pe[pf:L], slots[b][:pf], pf,
                                  int(reqs[b]), P, W, sm, D, chunk_mode="qdq", dtype=torch.float64)
        torch.testing.assert_close(out[s:e].double(), ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("D,R,H", [(512, 64, 16), (256, 32, 40)], ids=["dsv2", "minicpm3"])
def test_extend_output_independent_of_page_layout(D, R, H):
    """The same prefix tokens stored in other physical places (page sizes 64,
    16 and 1, other shuffles, other request indices) give the same extend
    output bits: the gather hands the attention the same rows in the same
    order."""
    from tests.helpers import alloc_slots
    P, W = 4, 16
    prefixes, chunks = [700, 0, 65], [40, 9, 70]
    n = sum(prefixes)
    sm = 1.0 / math.sqrt(96 if D == 256 else 192)
    x = synth.make_latent(n, D, 3, seed=81, device=DEV)
    pe = synth.make_normal((n, R), 82, device=DEV)
    rt = synth.make_rotation(D, 83).to(torch.bfloat16).t().contiguous().to(DEV)
    T = sum(chunks)
    q = synth.make_normal((T, H, D + R), 84, std=2.0 / (sm * math.sqrt(D + R))).to(DEV)
    kc = synth.make_normal((T, D + R), 85).to(DEV)
    qo = torch.tensor(np.concatenate([[0], np.cumsum(chunks)]), dtype=torch.int32, device=DEV)
    outs = []
    for page, seed, reqs in ((64, 5, [1, 2, 3]), (16, 6, [3, 1, 2]), (1, 7, [2, 3, 1])):
        slots, pages, num_slots = alloc_slots(prefixes, page, seed)
        max_reqs = len(prefixes) + 1
        hp_rows = 1 + max_reqs * (P + W)
        codes = torch.zeros(num_slots, D // 4, dtype=torch.uint8, device=DEV)
        params = torch.zeros(num_slots, D // 128, 2, dtype=torch.float32, device=DEV)
        rope = torch.zeros(num_slots, R, dtype=torch.bfloat16, device=DEV)
        hp = torch.zeros(hp_rows, D, dtype=torch.bfloat16, device=DEV)
        row = torch.full((num_slots,), -1, dtype=torch.int32, device=DEV)
        owner = torch.zeros(hp_rows, dtype=torch.int32, device=DEV)
        live = [b for b in range(len(prefixes)) if prefixes[b] > 0]
        loc = torch.from_numpy(np.concatenate([slots[b] for b in live])).to(DEV)
        pos = torch.from_numpy(np.concatenate([np.arange(prefixes[b]) for b in live])).to(DEV)
        seq = torch.from_numpy(np.concatenate([np.full(prefixes[b], prefixes[b]) for b in live])).to(DEV)
        rq = torch.from_numpy(np.concatenate([np.full(prefixes[b], reqs[b]) for b in live])).to(DEV)
        kernels.write_rows(x, pe, rt, loc, seq, pos, rq, codes, params, rope, hp, row, owner, P, W, max_reqs,
                           0.9810652732849121, 1.16)
        indptr, indices = index_lists(slots, pages, page)
        out = torch.full((T, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
        kernels.extend_fwd(q, kc, qo, indptr, indices, torch.tensor(prefixes, dtype=torch.int64, device=DEV),
                           torch.tensor(reqs, dtype=torch.int64, device=DEV), codes, params, rope, hp, max(chunks),
                           out, sm, P, W, page, max_reqs=max_reqs)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.isfinite(outs[0].float()).all()
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
