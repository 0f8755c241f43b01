"""HIP-graph capture of a full decode step (writer + split prep + packed decode).

Serving captures the decode step in a graph (deployment/serve.py:164) with a
padded batch: padding rows use slot 0, which must never claim a window row
(mla_fused_writer.py:41-43), and the decode scratch is sized for the captured
batch (rolaq_sglang.patch:62-111). The captured step is replayed over several
decode steps, with this program's own eager work (new inputs copied into the
static buffers) between replays; every replay must leave the pool and the
output exactly as the same step run eagerly on a twin pool, and the replayed
outputs of the live rows must match the oracle's dequantize-then-attention over
the rows the replays wrote (rtol 2e-2 / atol 2e-3).
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention
from mla_kv_quant_amd import PackedMLAPool, synth, writer
from mla_kv_quant_amd.decode import packed_mla_decode_gf_fwd, prepare_gf_splits
from tests.helpers import gpu_pool_to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_captured_decode_step_replays_match_eager():
    D, R, H, P, W, layers = 512, 64, 16, 4, 16, 2
    lengths0 = [40, 100, 7]
    nreq, Bg, steps, size, max_splits = len(lengths0), len(lengths0) + 1, 5, 512, 8
    rots = [synth.make_rotation(D, 300 + i) for i in range(layers)]

    def make_pool():
        return PackedMLAPool(size, layers, D, R, 8, P, W, device=DEV, rotations=rots)

    pools = {"graph": make_pool(), "eager": make_pool()}
    base = [1 + 150 * b for b in range(nreq)]  # request b owns slots base_b .. base_b + 149
    for li in range(layers):
        for b, L in enumerate(lengths0):
            loc = torch.arange(base[b], base[b] + L, device=DEV)
            x = synth.make_latent(L, D, 5, seed=10 * li + b).to(DEV)
            pe = synth.make_normal((L, R), 20 * li + b).to(DEV)
            for p in pools.values():
                writer.write_prefill(p, li, loc, x, pe, torch.arange(L, device=DEV), torch.full((L,), L, device=DEV),
                                     torch.full((L,), b + 1, device=DEV))

    sm = 1 / math.sqrt(192)
    maxtok = sum(lengths0) + nreq * steps + 1
    st = {  # static inputs of the captured step
        "loc": torch.zeros(Bg, dtype=torch.int64, device=DEV),
        "seq": torch.ones(Bg, dtype=torch.int64, device=DEV),
        "req": torch.zeros(Bg, dtype=torch.int64, device=DEV),
        "ckv": torch.zeros(layers, Bg, D, dtype=torch.bfloat16, device=DEV),
        "kpe": torch.zeros(layers, Bg, R, dtype=torch.bfloat16, device=DEV),
        "q": torch.zeros(layers, Bg, H, D + R, dtype=torch.bfloat16, device=DEV),
        "indptr": torch.zeros(Bg + 1, dtype=torch.int32, device=DEV),
        "indices": torch.zeros(maxtok, dtype=torch.int32, device=DEV),
        "ns": torch.full((Bg,), 4, dtype=torch.int32, device=DEV),
    }
    quant, merge = torch.empty_like(st["ns"]), torch.empty_like(st["ns"])
    outs = {k: {"logits": torch.empty(Bg, H, max_splits + 1, D, device=DEV),
                "lse": torch.empty(Bg, H, max_splits + 1, device=DEV),
                "o": torch.zeros(layers, Bg, H, D, dtype=torch.bfloat16, device=DEV)} for k in pools}

    def set_inputs(s):
        lens = [L + s + 1 for L in lengths0]
        loc = [base[b] + lens[b] - 1 for b in range(nreq)] + [0]          # padding row -> slot 0
        seq = lens + [1]
        req = [b + 1 for b in range(nreq)] + [0]
        idx = np.concatenate([np.arange(base[b], base[b] + lens[b]) for b in range(nreq)] + [np.zeros(1)])
        ptr = np.concatenate([[0], np.cumsum(lens + [1])])
        st["loc"].copy_(torch.tensor(loc))
        st["seq"].copy_(torch.tensor(seq))
        st["req"].copy_(torch.tensor(req))
        st["indices"][: len(idx)].copy_(torch.from_numpy(idx.astype(np.int32)))
        st["indptr"].copy_(torch.from_numpy(ptr.astype(np.int32)))
        st["ckv"].copy_(synth.make_latent(layers * Bg, D, 5, seed=500 + s).view(layers, Bg, D))
        st["kpe"].copy_(synth.make_normal((layers, Bg, R), 600 + s))
        st["q"].copy_(synth.make_normal((layers, Bg, H, D + R), 700 + s, std=2 / (sm * math.sqrt(D + R))))

    def step(pool, out):
        pool.set_window_meta(True, st["seq"], st["req"])
        prepare_gf_splits(st["ns"], quant, merge)
        for li in range(layers):
            assert writer.try_fast_decode_store(pool, li, st["loc"], st["ckv"][li], st["kpe"][li])
            packed_mla_decode_gf_fwd(st["q"][li], out["o"][li], pool, li, st["indptr"], st["indices"], st["ns"],
                                     max_splits, out["logits"], out["lse"], sm, seq_lens=st["seq"],
                                     req_pool_indices=st["req"])

    set_inputs(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(pools["graph"], outs["graph"])  # warm-up (caches the bf16 rotations)
    torch.cuda.current_stream().wait_stream(side)
    step(pools["eager"], outs["eager"])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(pools["graph"], outs["graph"])

    for s in range(steps):
        set_inputs(s)
        graph.replay()
        step(pools["eager"], outs["eager"])
        torch.cuda.synchronize()
        og, oe = outs["graph"]["o"], outs["eager"]["o"]
        assert torch.isfinite(og[:, :nreq].float()).all()
        assert torch.equal(og, oe), f"replay {s}: output differs from the eager step"
        pg, pe_ = pools["graph"], pools["eager"]
        for li in range(layers):
            for name in ("c_codes", "c_params", "rope_buf", "hp_c"):
                assert torch.equal(getattr(pg, name)[li], getattr(pe_, name)[li]), (s, li, name)
        assert torch.equal(pg.hp_row_of_slot, pe_.hp_row_of_slot)
        assert torch.equal(pg.hp_owner_of_row, pe_.hp_owner_of_row)
        # slot 0 (graph padding) never claims a window row
        assert int(pg.hp_row_of_slot[0]) == -1
        # the replayed outputs of the live rows against the oracle's
        # dequantize-then-attention over the rows the replays wrote
        lens = [L + s + 1 for L in lengths0]
        slots = [np.arange(base[b], base[b] + lens[b]) for b in range(nreq)]
        for li in range(layers):
            pool_np = gpu_pool_to_oracle({"codes": pg.c_codes[li], "params": pg.c_params[li], "rope": pg.rope_buf[li],
                                          "hp": pg.hp_c[li], "row_of_slot": pg.hp_row_of_slot,
                                          "owner_of_row": pg.hp_owner_of_row})
            qh = st["q"][li, :nreq].float().cpu()
            ref, _ = attention.decode(pool_np, qh[..., :D], qh[..., D:], slots, lens, list(range(1, nreq + 1)), P, W,
                                      sm, D, "stored64", max_reqs=8)
            torch.testing.assert_close(og[li, :nreq].float().cpu().double(), ref, rtol=2e-2, atol=2e-3)
