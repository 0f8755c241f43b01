"""Pin the oracle's absorbed attention, split merge and extend (CPU only)."""

import math

import numpy as np
import pytest
import torch

from oracle import attention, codec, layout, window
from mla_kv_quant_amd import synth


def brute_force(q_lat, q_rope, k_lat, k_rope, scale):
    """Pure-Python float64 attention for one query head (tiny inputs only)."""
    L = len(k_lat)
    s = [scale * (sum(a * b for a, b in zip(q_lat, k_lat[t])) + sum(a * b for a, b in zip(q_rope, k_rope[t])))
         for t in range(L)]
    m = max(s)
    w = [math.exp(v - m) for v in s]
    z = sum(w)
    return [sum(w[t] * k_lat[t][d] for t in range(L)) / z for d in range(len(k_lat[0]))], m + math.log(z)


def test_attend_matches_brute_force():
    g = torch.Generator().manual_seed(0)
    L, H, D, R = 9, 2, 16, 4
    ql, qr = torch.randn(1, H, D, generator=g, dtype=torch.float64), torch.randn(1, H, R, generator=g, dtype=torch.float64)
    kl, kr = torch.randn(L, D, generator=g, dtype=torch.float64), torch.randn(L, R, generator=g, dtype=torch.float64)
    out, lse = attention.attend(ql, qr, kl, kr, 0.3, torch.float64)
    for h in range(H):
        o, l = brute_force(ql[0, h].tolist(), qr[0, h].tolist(), kl.tolist(), kr.tolist(), 0.3)
        assert np.allclose(out[0, h].numpy(), o, rtol=1e-12, atol=1e-12)
        assert lse[0, h].item() == pytest.approx(l, rel=1e-12)


def test_split_merge_equals_unsplit_and_empty_is_neutral():
    g = torch.Generator().manual_seed(1)
    L, H, D, R = 100, 3, 32, 8
    ql, qr = torch.randn(1, H, D, generator=g, dtype=torch.float64), torch.randn(1, H, R, generator=g, dtype=torch.float64)
    kl, kr = torch.randn(L, D, generator=g, dtype=torch.float64), torch.randn(L, R, generator=g, dtype=torch.float64)
    full, _ = attention.attend(ql, qr, kl, kr, 0.2, torch.float64)
    for bounds in ([(0, 100)], [(0, 37), (37, 100)], [(0, 10), (10, 10), (10, 64), (64, 100), (100, 100)]):
        parts, lses = attention.split_partials(ql, qr, kl, kr, 0.2, bounds)
        merged = attention.merge_splits(parts, lses)
        assert torch.allclose(merged, full, rtol=1e-12, atol=1e-12)


def test_absorbed_form_is_rotation_invariant():
    # attention in the rotated frame (q R, c R) equals the un-rotated one, output rotated
    g = torch.Generator().manual_seed(2)
    D, R, L, H = 128, 8, 20, 4
    q, r = torch.linalg.qr(torch.randn(D, D, generator=g, dtype=torch.float64))
    rot = q * torch.sign(torch.diagonal(r))[None, :]  # exactly orthogonal in float64
    ql, qr = torch.randn(1, H, D, generator=g, dtype=torch.float64), torch.randn(1, H, R, generator=g, dtype=torch.float64)
    kl, kr = torch.randn(L, D, generator=g, dtype=torch.float64), torch.randn(L, R, generator=g, dtype=torch.float64)
    o, lse = attention.attend(ql, qr, kl, kr, 0.1, torch.float64)
    o_r, lse_r = attention.attend(ql @ rot, qr, kl @ rot, kr, 0.1, torch.float64)
    assert torch.allclose(o_r, o @ rot, atol=1e-10)
    assert torch.allclose(lse_r, lse, atol=1e-10)


def _pool_with_sequence(L, D, R, P, W, seed, req=1, page=16, max_reqs=4):
    pool = window.new_pool(1 + 4 * ((L + page - 1) // page) * page, D, R, max_reqs, P, W)
    pages = np.random.default_rng(seed).permutation(np.arange(1, 1 + 4 * ((L + page - 1) // page)))[: (L + page - 1) // page]
    slots = (pages[:, None] * page + np.arange(page)[None, :]).reshape(-1)[:L]
    rot = synth.make_rotation(D, seed)
    x = synth.make_latent(L, D, 2, seed=seed + 1)
    pe = synth.make_normal((L, R), seed + 2)
    c = window.write_rows(pool, x, pe, slots, np.full(L, L), np.full(L, req), rot, 0.98, 1.16,
                          P, W, max_reqs, positions=np.arange(L))
    return pool, slots, c, pe


def test_gather_rows_window_and_quantized():
    D, R, P, W, L = 256, 32, 4, 16, 50
    pool, slots, c, pe = _pool_with_sequence(L, D, R, P, W, seed=5)
    lat, rope = attention.gather_rows(pool, slots, 1, L, P, W, D, round_bf16=True)
    _, _, _, qdq = codec.lloyd_codec(c, 128, 0.98, 1.16)
    for t in range(L):
        if t < P or t >= L - W:
            assert torch.equal(lat[t], c[t].to(torch.bfloat16).float())
        else:
            assert torch.equal(lat[t], qdq[t].to(torch.bfloat16).float())
    assert torch.equal(rope, pe.float())


def test_decode_flavours_agree():
    D, R, P, W, L, H = 256, 32, 4, 16, 70, 4
    pool, slots, c, _ = _pool_with_sequence(L, D, R, P, W, seed=9)
    q_lat = synth.make_normal((1, H, D), 1, std=0.3)
    q_rope = synth.make_normal((1, H, R), 2, std=0.3)
    o64, lse64 = attention.decode(pool, q_lat, q_rope, [slots], [L], [1], P, W, 0.1, D, "fp64")
    o32, _ = attention.decode(pool, q_lat, q_rope, [slots], [L], [1], P, W, 0.1, D, "fp32")
    oe, _ = attention.decode(pool, q_lat, q_rope, [slots], [L], [1], P, W, 0.1, D, "bf16_eager")
    assert torch.allclose(o32.double(), o64, rtol=2e-2, atol=2e-3)
    assert torch.allclose(oe.double(), o64, rtol=5e-2, atol=1e-2)


@pytest.mark.parametrize("T,L,causal", [(1, 70, False), (9, 40, True)])
def test_bf16_eager_equals_transformers_eager_attention(T, L, causal):
    """attend_bf16_eager is the reference model's attention in bf16: transformers'
    eager_attention_forward (models/deepseek_v2/modeling_deepseek_v2.py, the
    function the reference's HF path runs) with the absorbed query, one shared
    key/value head repeated over the heads (MQA), bit for bit."""
    from types import SimpleNamespace

    from transformers.models.deepseek_v2.modeling_deepseek_v2 import eager_attention_forward

    D, R, H, sm = 64, 16, 5, 0.13
    ql = synth.make_normal((T, H, D), 31, std=1.3)
    qr = synth.make_normal((T, H, R), 32, std=1.3)
    kl = synth.make_latent(L, D, 2, seed=33).float()
    kr = synth.make_normal((L, R), 34).float()
    mask = None
    if causal:
        mask = torch.arange(L)[None, :] <= torch.arange(L - T, L)[:, None]
    ours = attention.attend_bf16_eager(ql, qr, kl, kr, sm, mask=mask)
    query = torch.cat([ql, qr], -1).to(torch.bfloat16).transpose(0, 1)[None]  # [1, H, T, D + R]
    key = torch.cat([kl, kr], -1).to(torch.bfloat16)[None, None]              # [1, 1, L, D + R]
    value = kl.to(torch.bfloat16)[None, None]                                  # [1, 1, L, D]
    add = None
    if mask is not None:
        add = torch.zeros(1, 1, T, L, dtype=torch.bfloat16).masked_fill(~mask[None, None], float("-inf"))
    module = SimpleNamespace(num_key_value_groups=H, training=False)
    ref, _ = eager_attention_forward(module, query, key, value, add, sm)
    assert torch.equal(ours, ref[0])


def test_extend_causal_and_window():
    D, R, P, W, H = 256, 32, 4, 16, 2
    prefix, Tq = 40, 8
    pool, slots, c, pe = _pool_with_sequence(prefix, D, R, P, W, seed=13)
    ql = synth.make_normal((Tq, H, D), 1, std=0.2)
    qr = synth.make_normal((Tq, H, R), 2, std=0.2)
    chunk = synth.make_normal((Tq, D), 3)
    chunk_r = synth.make_normal((Tq, R), 4)
    out, lse = attention.extend(pool, ql, qr, chunk, chunk_r, slots, prefix, 1, P, W, 0.1, D,
                                dtype=torch.float64)
    # query i sees prefix + chunk rows 0..i: compare with an explicit per-query decode
    lat_p, rope_p = attention.gather_rows(pool, slots, 1, prefix, P, W, D)
    # Tq < W: prefix rows prefix+Tq-W .. prefix-1 stay BF16, earlier ones left the window
    lat_q, _ = attention.gather_rows(pool, slots, 1, prefix, 0, 0, D)
    for t in range(prefix):
        if P <= t < prefix + Tq - W:
            lat_p[t] = lat_q[t]
    for i in range(Tq):
        kl = torch.cat([lat_p, chunk[: i + 1].float()])
        kr = torch.cat([rope_p, chunk_r[: i + 1].float()])
        o, _ = attention.attend(ql[i:i + 1].double(), qr[i:i + 1].double(), kl, kr, 0.1, torch.float64)
        assert torch.allclose(out[i], o[0], atol=1e-10)
