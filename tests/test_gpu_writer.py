"""GPU parity: quantize/pack and the fused writer against the CPU oracle."""

import numpy as np
import pytest
import torch

import math

from oracle import attention, codec, layout, window
from mla_kv_quant_amd import PackedMLAPool, synth, writer
from mla_kv_quant_amd.decode import packed_mla_decode_gf_fwd
from tests.helpers import bf16_np_to_torch, make_queries

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _codes_close(gpu_codes: np.ndarray, ref_codes: np.ndarray, budget: float):
    diff = gpu_codes.astype(np.int16) - ref_codes.astype(np.int16)
    bad = np.count_nonzero(diff)
    assert np.abs(diff).max(initial=0) <= 1, "a code differs by more than one level"
    assert bad <= budget * diff.size, f"{bad} of {diff.size} codes differ (budget {budget})"
    return bad


@pytest.mark.parametrize("D", [512, 256])
@pytest.mark.parametrize("tg", [(codec.LLOYD_MAX_THRESHOLD, 1.16), (0.75, None), (1.2, None)])
def test_scatter_pack_rows_matches_oracle(D, tg):
    t, g = tg
    g = codec.signal_gain(t) if g is None else g
    n = 4096 if D == 512 else 2048
    rot = synth.make_rotation(D, 5)
    x = codec.rotate(synth.make_latent(n, D, 8, seed=D), rot)
    x[0] = 3.25                               # constant row: std = 1e-4
    x[1, ::2], x[1, 1::2] = 1.0, -1.0         # +-1 alternating
    x[2] = torch.linspace(-4, 4, D)
    x[3] = 0.0
    S = n + 500
    slots = torch.from_numpy(np.random.default_rng(1).permutation(np.arange(1, S))[:n].astype(np.int32))
    codes = torch.zeros(S, D // 4, dtype=torch.uint8, device=DEV)
    params = torch.zeros(S, D // 128, 2, dtype=torch.float32, device=DEV)
    writer.scatter_pack_rows(x.to(DEV), slots.to(DEV), codes, params, 128, True, 2, (t, g) if tg[1] is None else None)
    torch.cuda.synchronize()
    ref_codes, ref_scale, ref_zero, _ = codec.lloyd_codec(x, 128, t, codec.snap_gain(g))
    got = codes.cpu().numpy()[slots.numpy()]
    gpu_codes = layout.unpack_codes(got, D)
    nbad = _codes_close(gpu_codes, ref_codes.numpy(), 1e-5)
    # byte layout: rows whose codes agree pack to exactly the oracle's bytes
    same = (gpu_codes == ref_codes.numpy()).all(axis=1)
    assert same.sum() >= n - nbad
    assert np.array_equal(got[same], layout.pack_codes(ref_codes.numpy()[same]))
    p = params.cpu()[slots.long()]
    torch.testing.assert_close(p[..., 0], ref_scale, rtol=2e-6, atol=0)
    torch.testing.assert_close(p[..., 1], ref_zero, rtol=1e-5, atol=1e-5)
    # slots not written stay zero; slot 0 untouched
    mask = np.ones(S, bool)
    mask[slots.numpy()] = False
    assert not codes.cpu().numpy()[mask].any() and not params.cpu().numpy()[mask].any()


def test_scatter_pack_rows_errors_and_empty():
    x = torch.zeros(0, 512, device=DEV)
    codes = torch.zeros(4, 128, dtype=torch.uint8, device=DEV)
    params = torch.zeros(4, 4, 2, device=DEV)
    writer.scatter_pack_rows(x, torch.zeros(0, dtype=torch.int32, device=DEV), codes, params, 128, True)
    with pytest.raises(ValueError):
        writer.scatter_pack_rows(torch.zeros(2, 512, device=DEV), torch.ones(2, dtype=torch.int32, device=DEV),
                                 codes, params, 128, False, 2, (0.9, 1.1))
    assert not codes.any()


def _oracle_pool_from(pool: PackedMLAPool, li: int):
    D, R = pool.kv_lora_rank, pool.qk_rope_head_dim
    o = window.new_pool(pool.size + 1, D, R, pool._max_reqs, pool._win_p, pool._win_r)
    return o


def _compare_layer(pool: PackedMLAPool, li: int, ref: dict, written: np.ndarray, flips: float):
    D = pool.kv_lora_rank
    codes = pool.c_codes[li].cpu().numpy()
    _codes_close(layout.unpack_codes(codes[written], D), layout.unpack_codes(ref["codes"][written], D), flips)
    torch.testing.assert_close(pool.c_params[li].cpu()[written][..., 0], torch.from_numpy(ref["params"][written][..., 0]),
                               rtol=1e-5, atol=0)
    torch.testing.assert_close(pool.c_params[li].cpu()[written][..., 1], torch.from_numpy(ref["params"][written][..., 1]),
                               rtol=1e-4, atol=1e-4)
    assert np.array_equal(pool.rope_buf[li].cpu().view(torch.int16).numpy().view(np.uint16), ref["rope"])
    hp = pool.hp_c[li].cpu().float()
    torch.testing.assert_close(hp, bf16_np_to_torch(ref["hp"]).float(), rtol=2 ** -7, atol=1e-6)
    assert np.array_equal(pool.hp_row_of_slot.cpu().numpy(), ref["row_of_slot"])
    assert np.array_equal(pool.hp_owner_of_row.cpu().numpy(), ref["owner_of_row"])


@pytest.mark.parametrize("D,R", [(512, 64), (256, 32)])
def test_fused_writer_prefill_then_decode(D, R):
    P, W, max_reqs, layers = 4, 16, 6, 2
    lengths = [1, 3, 20, 21, 300, 777]
    size = 4096
    rots = [synth.make_rotation(D, 100 + i) for i in range(layers)]
    quant = [None, (0.8, codec.signal_gain(0.8))]
    pool = PackedMLAPool(size, layers, D, R, max_reqs, P, W, device=DEV, rotations=rots, quantizers=quant)
    refs = [window.new_pool(size + 1, D, R, max_reqs, P, W) for _ in range(layers)]
    rng = np.random.default_rng(0)
    free = list(rng.permutation(np.arange(1, size + 1)))
    seq_slots = []
    # prefill: one chunk per request, positions 0..L-1
    for li in range(layers):
        t, g = quant[li] if quant[li] else (writer.LM_THRESHOLD, writer.LM_GAIN)
        for b, L in enumerate(lengths):
            if li == 0:
                seq_slots.append([int(free.pop()) for _ in range(L)])
            loc = np.array(seq_slots[b], np.int64)
            x = synth.make_latent(L, D, 5, seed=1000 * li + b)
            pe = synth.make_normal((L, R), 2000 * li + b)
            window.write_rows(refs[li], x, pe, loc, np.full(L, L), np.full(L, b + 1), rots[li], t, g,
                              P, W, max_reqs, positions=np.arange(L))
            writer.write_prefill(pool, li, torch.from_numpy(loc).to(DEV), x.to(DEV), pe.to(DEV),
                                 torch.arange(L, device=DEV), torch.full((L,), L, device=DEV),
                                 torch.full((L,), b + 1, device=DEV))
    torch.cuda.synchronize()
    written = np.concatenate([np.array(s) for s in seq_slots])
    for li in range(layers):
        _compare_layer(pool, li, refs[li], written, 1e-4)
    # decode steps: every request appends one token per step; slot 0 pads the batch
    for step in range(3):
        seq = np.array([L + step + 1 for L in lengths] + [1], np.int64)
        new = [int(free.pop()) for _ in lengths] + [0]
        req = np.array([b + 1 for b in range(len(lengths))] + [0], np.int64)
        for b in range(len(lengths)):
            seq_slots[b].append(new[b])
        pool.set_window_meta(True, torch.from_numpy(seq).to(DEV), torch.from_numpy(req).to(DEV))
        for li in range(layers):
            t, g = quant[li] if quant[li] else (writer.LM_THRESHOLD, writer.LM_GAIN)
            x = synth.make_latent(len(seq), D, 5, seed=5000 + 10 * step + li)
            pe = synth.make_normal((len(seq), R), 6000 + 10 * step + li)
            window.write_rows(refs[li], x, pe, np.array(new), seq, req, rots[li], t, g, P, W, max_reqs)
            assert writer.try_fast_decode_store(pool, li, torch.tensor(new, device=DEV), x.to(DEV), pe.to(DEV))
        torch.cuda.synchronize()
        written = np.concatenate([np.array(s) for s in seq_slots])
        for li in range(layers):
            _compare_layer(pool, li, refs[li], written, 1e-4)
    # decode over what the GPU writer stored, against the oracle over its own pool
    # (requests below max_reqs: the last one has no ring rows; token slots)
    H = 16
    sm = 1.0 / math.sqrt(192 if D == 512 else 96)
    nb = max_reqs - 1
    lens = [L + 3 for L in lengths][:nb]
    slots = [np.array(s, np.int64) for s in seq_slots][:nb]
    q = make_queries(nb, H, D, R, sm, seed=9)
    indptr = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    indices = torch.from_numpy(np.concatenate(slots).astype(np.int32)).to(DEV)
    for li in range(layers):
        o = torch.empty(nb, H, D, dtype=torch.bfloat16, device=DEV)
        logits = torch.empty(nb, H, 9, D, device=DEV)
        lse = torch.empty(nb, H, 9, device=DEV)
        packed_mla_decode_gf_fwd(q.to(DEV), o, pool, li, indptr, indices,
                                 torch.tensor([2, 3, 1, 4, 8], dtype=torch.int32, device=DEV), 8, logits, lse, sm,
                                 seq_lens=torch.tensor(lens, device=DEV),
                                 req_pool_indices=torch.arange(1, nb + 1, device=DEV))
        torch.cuda.synchronize()
        ref64, _ = attention.decode(refs[li], q[..., :D], q[..., D:], slots, lens, list(range(1, nb + 1)), P, W, sm,
                                    D, "stored64", max_reqs=max_reqs)
        # the GPU pool may differ from the oracle's by rare +-1 codes (the budget above)
        torch.testing.assert_close(o.float().cpu().double(), ref64, rtol=2e-2, atol=2e-3)


def test_fused_writer_unrotated_layer_and_fallbacks():
    D, R, P, W = 512, 64, 4, 16
    pool = PackedMLAPool(64, 1, D, R, 4, P, W, device=DEV, rotations=[None])
    ref = window.new_pool(65, D, R, 4, P, W)
    x = synth.make_latent(3, D, 5, seed=9)
    pe = synth.make_normal((3, R), 10)
    seq, req, loc = np.array([5, 30, 2]), np.array([1, 2, 3]), np.array([7, 8, 9])
    window.write_rows(ref, x, pe, loc, seq, req, None, writer.LM_THRESHOLD, writer.LM_GAIN, P, W, 4)
    # fallback: not a decode step / flagged / budget -> False and nothing written
    for meta in ((False, False), (True, True)):
        pool.set_window_meta(meta[0], torch.from_numpy(seq).to(DEV), torch.from_numpy(req).to(DEV), fallback=meta[1])
        assert not writer.try_fast_decode_store(pool, 0, torch.from_numpy(loc).to(DEV), x.to(DEV), pe.to(DEV))
    pool.set_window_meta(True, torch.from_numpy(seq[:2]).to(DEV), torch.from_numpy(req[:2]).to(DEV))
    assert not writer.try_fast_decode_store(pool, 0, torch.from_numpy(loc).to(DEV), x.to(DEV), pe.to(DEV))
    pool.set_window_meta(True, torch.from_numpy(seq).to(DEV), torch.from_numpy(req).to(DEV))
    pool._selfcheck_budget = 1
    assert not writer.try_fast_decode_store(pool, 0, torch.from_numpy(loc).to(DEV), x.to(DEV), pe.to(DEV))
    torch.cuda.synchronize()
    assert not pool.c_codes[0].any() and not pool.rope_buf[0].view(torch.int16).any()
    pool._selfcheck_budget = 0
    assert writer.try_fast_decode_store(pool, 0, torch.from_numpy(loc).to(DEV), x.to(DEV), pe.to(DEV))
    torch.cuda.synchronize()
    _compare_layer(pool, 0, ref, loc, 1e-5)


def test_writer_request_index_beyond_32_bits_has_no_ring_rows():
    """req_idx is int64: an index whose low 32 bits name a valid request but
    which does not fit 32 bits is outside [0, max_reqs) (mla_fused_writer.py:41)
    and claims no ring row; the codes are written as for any row."""
    from mla_kv_quant_amd import kernels

    D, R, P, W, max_reqs, n = 512, 64, 4, 16, 4, 40
    rot = synth.make_rotation(D, 3).to(torch.bfloat16).t().contiguous().to(DEV)
    x = synth.make_latent(n, D, 5, seed=4, device=DEV)
    pe = synth.make_normal((n, R), 5, device=DEV)
    loc = torch.arange(1, n + 1, device=DEV)
    pos = torch.arange(n, device=DEV)
    seq = torch.full((n,), n, device=DEV)
    outs = []
    for rq in (-1, (1 << 32) + 1):
        bufs = {
            "codes": torch.zeros(n + 1, D // 4, dtype=torch.uint8, device=DEV),
            "params": torch.zeros(n + 1, D // 128, 2, device=DEV),
            "rope": torch.zeros(n + 1, R, dtype=torch.bfloat16, device=DEV),
            "hp": torch.zeros(1 + max_reqs * (P + W), D, dtype=torch.bfloat16, device=DEV),
            "row": torch.full((n + 1,), -7, dtype=torch.int32, device=DEV),
            "owner": torch.zeros(1 + max_reqs * (P + W), dtype=torch.int32, device=DEV),
        }
        kernels.write_rows(x, pe, rot, loc, seq, pos, torch.full((n,), rq, dtype=torch.int64, device=DEV),
                           bufs["codes"], bufs["params"], bufs["rope"], bufs["hp"], bufs["row"], bufs["owner"],
                           P, W, max_reqs, 0.9810652732849121, 1.16)
        torch.cuda.synchronize()
        outs.append(bufs)
    a, b = outs
    assert not b["hp"].view(torch.int16).any() and not b["owner"].any()
    assert (b["row"][1:] == -1).all()
    for k in ("codes", "params", "rope", "row"):
        assert torch.equal(a[k], b[k]), k


@pytest.mark.parametrize("D,R", [(512, 64), (256, 32)])
def test_row_local_batching_is_exact(D, R):
    """The quantizer is row-local (mla_quant/cache.py:188-202,1142-1159): one
    launch over 200K rows and launches over random slices of them (tile and
    stripe boundaries anywhere) store the same bytes in every pool buffer."""
    P, W = 4, 16
    lengths = [1, 17, 1000, 64 * 1000 + 3, 2049, 130_000 - 70]
    n = sum(lengths)
    size = n + 8
    max_reqs = len(lengths) + 1
    rot = [synth.make_rotation(D, 401)]
    quant = [(0.9, codec.signal_gain(0.9))]
    pools = [PackedMLAPool(size, 1, D, R, max_reqs, P, W, device=DEV, rotations=rot, quantizers=quant)
             for _ in range(2)]
    rng = np.random.default_rng(403)
    loc = torch.from_numpy(rng.permutation(np.arange(1, size + 1))[:n].astype(np.int64)).to(DEV)
    pos = torch.cat([torch.arange(L, device=DEV) for L in lengths])
    seq = torch.cat([torch.full((L,), L, device=DEV) for L in lengths])
    req = torch.cat([torch.full((L,), i + 1, device=DEV) for i, L in enumerate(lengths)])
    x = synth.make_latent(n, D, 5, seed=404, device=DEV)
    pe = synth.make_normal((n, R), 405, device=DEV)
    writer.write_prefill(pools[0], 0, loc, x, pe, pos, seq, req)
    cuts = [0, *sorted(rng.choice(np.arange(1, n), size=9, replace=False).tolist()), n]
    for a, b in zip(cuts[:-1], cuts[1:]):
        writer.write_prefill(pools[1], 0, loc[a:b], x[a:b], pe[a:b], pos[a:b], seq[a:b], req[a:b])
    torch.cuda.synchronize()
    for name in ("c_codes", "c_params", "rope_buf", "hp_c"):
        u, v = getattr(pools[0], name)[0], getattr(pools[1], name)[0]
        assert torch.equal(u.view(torch.uint8), v.view(torch.uint8)), name
    assert torch.equal(pools[0].hp_row_of_slot, pools[1].hp_row_of_slot)
    assert torch.equal(pools[0].hp_owner_of_row, pools[1].hp_owner_of_row)
    assert int((pools[0].hp_row_of_slot >= 0).sum()) == sum(min(L, P + W) for L in lengths)
