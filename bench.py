"""Benchmark of the packed-INT2 RoLaQ MLA path on one MI355X.

Headline (``value``): absorbed MLA decode attention over the INT2 cache at
BASELINE config 2 -- batch 32 x 16384 context, 16 heads, latent 512, rope 64,
s4r16 BF16 window, page 64 -- in microseconds per layer. A step is one decode
pass over 27 layers, each with its own cache buffers (every layer's ~151 MB
working set, so the 256 MB MALL cannot serve repeats). The cache is written
beforehand by this library's fused writer from synthetic latents (N(0,1), 1%
outlier channels x20, seeded rotation per layer).

Also reported (``writer``): the fused cache writer at config 1 -- 64 sequences
x 2048-token prefill chunk, 27 layers with their own buffers -- in Mtokens/s
(token-layers per second) and as a fraction of HBM peak.

Also reported (``reported``): decode at config 3 (batch 128, ragged context
U[2048, 8192], shuffled pages) and config 4a (MiniCPM3 shape: 40 heads, latent
256, batch 64 x 16384), 4 layers each with their own buffers.

``roofline``: algorithmic bytes per decode layer (288 B per INT2 token, window
rows, q and out) over the measured layer time, against 8 TB/s. ``traffic`` is
taken from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary when present.
``cpu_baseline``: the reference arithmetic restated in PyTorch (the oracle) on
the host cores -- cfg0 codec + QDQ, a cfg1 layer of rotation + QDQ, a layer of
dequantize-then-attention at cfg2 (``value``) and cfg4a -- median of 5 runs on
bounded samples scaled to the full workload, with nproc and the CPU model.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=27)
    ap.add_argument("--splits", type=int, default=0, help="num_kv_splits per request (0 = pick the fastest)")
    ap.add_argument("--no-writer", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--writer-only", action="store_true", help="only the cfg1 writer (prints its own JSON)")
    ap.add_argument("--extend-only", action="store_true", help="only the cfg4b extend (prints its own JSON)")
    ap.add_argument("--no-extend", action="store_true")
    ap.add_argument("--no-reported", action="store_true", help="skip the cfg3 / cfg4a decode lines")
    ap.add_argument("--reported-only", action="store_true", help="only the cfg3 / cfg4a decode lines")
    ap.add_argument("--read-probe", action="store_true",
                    help="only time a sum over 4 GiB (the achievable read-only HBM rate)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only time a 1 GiB device copy (the reference kernel for rocprofv3 byte counters)")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# config 2: decode
# ---------------------------------------------------------------------------
class DecodeBench:
    """A decode workload: per-layer caches written by the fused writer, a shuffled page table."""

    B, L, H, D, R, P, W, PAGE = 32, 16384, 16, 512, 64, 4, 16, 64

    def __init__(self, layers: int, dev: str, B: int | None = None, lengths=None, H: int | None = None,
                 D: int | None = None, R: int | None = None, seed: int = 0):
        from mla_kv_quant_amd import kernels, synth

        self.B = B or self.B
        self.H, self.D, self.R = H or self.H, D or self.D, R or self.R
        self.layers, self.dev = layers, dev
        B, D, R, P, W, PAGE = self.B, self.D, self.R, self.P, self.W, self.PAGE
        self.lengths = np.asarray(lengths if lengths is not None else [self.L] * B, dtype=np.int64)
        self.L = int(self.lengths.max())
        pages_per_seq = (self.lengths + PAGE - 1) // PAGE
        npages = int(pages_per_seq.sum())
        rng = np.random.default_rng(seed)
        perm = rng.permutation(np.arange(1, npages + 1)).astype(np.int64)  # page 0 = padding
        indptr = np.concatenate([[0], np.cumsum(pages_per_seq)])
        self.num_slots = (npages + 1) * PAGE
        self.kv_indptr = torch.from_numpy(indptr.astype(np.int32)).to(dev)
        self.kv_indices = torch.from_numpy(perm.astype(np.int32)).to(dev)
        self.seq_lens = torch.from_numpy(self.lengths).to(dev)
        self.req = torch.arange(1, B + 1, dtype=torch.int64, device=dev)
        loc = torch.cat([(torch.from_numpy(perm[indptr[b]:indptr[b + 1]]).to(dev)[:, None] * PAGE
                          + torch.arange(PAGE, device=dev)).reshape(-1)[: self.lengths[b]] for b in range(B)])
        positions = torch.cat([torch.arange(int(n), device=dev) for n in self.lengths])
        lens_t = torch.from_numpy(self.lengths).to(dev)
        seqs = lens_t.repeat_interleave(lens_t)
        reqs = self.req.repeat_interleave(lens_t)
        n = int(self.lengths.sum())
        max_reqs = B + 1
        hp_rows = 1 + max_reqs * (P + W)
        self.caches = []
        self.sm_scale = 1.0 / math.sqrt(192 if D == 512 else 96)
        sigma = 2.0 / (self.sm_scale * math.sqrt(D + R))
        for layer in range(layers):
            c = {
                "codes": torch.zeros(self.num_slots, D // 4, dtype=torch.uint8, device=dev),
                "params": torch.zeros(self.num_slots, D // 128, 2, dtype=torch.float32, device=dev),
                "rope": torch.zeros(self.num_slots, R, dtype=torch.bfloat16, device=dev),
                "hp": torch.zeros(hp_rows, D, dtype=torch.bfloat16, device=dev),
                "row": torch.full((self.num_slots,), -1, dtype=torch.int32, device=dev),
                "owner": torch.zeros(hp_rows, dtype=torch.int32, device=dev),
            }
            rt = synth.layer_rotation(D, layer).to(torch.bfloat16).t().contiguous().to(dev)
            x = synth.make_latent(n, D, max(1, D // 100), seed=10_000 + layer, device=dev)
            pe = synth.make_normal((n, R), 20_000 + layer, device=dev)
            kernels.write_rows(x, pe, rt, loc, seqs, positions, reqs, c["codes"], c["params"], c["rope"],
                               c["hp"], c["row"], c["owner"], P, W, max_reqs,
                               synth.DEFAULT_THRESHOLD, synth.DEFAULT_GAIN)
            del x, pe
            c["q"] = synth.make_normal((B, self.H, D + R), 30_000 + layer, std=sigma, device=dev)
            self.caches.append(c)
        torch.cuda.synchronize()
        self.out = torch.empty(B, self.H, D, dtype=torch.bfloat16, device=dev)

    def alloc_scratch(self, max_splits: int):
        self.max_splits = max_splits
        self.logits = torch.empty(self.B, self.H, max_splits + 1, self.D, device=self.dev)
        self.lse = torch.empty(self.B, self.H, max_splits + 1, device=self.dev)

    def set_splits(self, ns: int):
        self.ns = torch.full((self.B,), ns, dtype=torch.int32, device=self.dev)

    def step(self):
        from mla_kv_quant_amd import kernels

        for c in self.caches:
            kernels.decode_fwd(c["q"], c["codes"], c["params"], c["rope"], c["hp"], self.kv_indptr,
                               self.kv_indices, self.seq_lens, self.req, self.ns, self.max_splits,
                               self.logits, self.lse, self.out, self.sm_scale, self.P, self.W, self.PAGE)

    def step_partials(self):
        """Stage 1 alone (the dominant kernel), one launch per layer."""
        from mla_kv_quant_amd import kernels

        for c in self.caches:
            kernels.decode_partials(c["q"], c["codes"], c["params"], c["rope"], c["hp"], self.kv_indptr,
                                    self.kv_indices, self.seq_lens, self.req, self.ns, self.max_splits,
                                    self.logits, self.lse, self.sm_scale, self.P, self.W, self.PAGE)

    def bytes_per_layer(self, with_out: bool = True) -> float:
        """Algorithmic bytes: D/4 + 8 NG + 2 R per INT2 token (288 B at D=512), window rows, q (and the output)."""
        B, P, W, D, R, H = self.B, self.P, self.W, self.D, self.R, self.H
        lens = self.lengths
        win = np.minimum(lens, P + W)
        int2 = int((lens - win).sum()) * (D // 4 + 8 * (D // 128) + 2 * R)
        window = int(win.sum()) * (2 * D + 2 * R)
        q_out = B * H * (D + R) * 2 + (B * H * D * 2 if with_out else 0)
        return float(int2 + window + q_out)

    def flops_per_layer(self) -> float:
        return float(2 * int(self.lengths.sum()) * self.H * (2 * self.D + self.R))


def time_loop(fn, steps: int, warmup: int) -> float:
    """Milliseconds per step: events on the current stream around exactly ``steps`` steps."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


# ---------------------------------------------------------------------------
# config 1: writer
# ---------------------------------------------------------------------------
class WriterBench:
    SEQS, CHUNK, D, R, P, W, PAGE = 64, 2048, 512, 64, 4, 16, 64

    def __init__(self, layers: int, dev: str):
        from mla_kv_quant_amd import synth

        self.layers, self.dev = layers, dev
        S, C, D, R, P, W, PAGE = self.SEQS, self.CHUNK, self.D, self.R, self.P, self.W, self.PAGE
        n = S * C
        self.n = n
        pages = np.random.default_rng(1).permutation(np.arange(1, S * (C // PAGE) + 1)).reshape(S, C // PAGE)
        slots = (torch.from_numpy(pages).to(dev)[:, :, None] * PAGE + torch.arange(PAGE, device=dev)).reshape(-1)
        self.loc = slots.contiguous()
        self.positions = torch.arange(C, device=dev).repeat(S)
        self.seqs = torch.full((n,), C, dtype=torch.int64, device=dev)
        self.reqs = torch.arange(1, S + 1, dtype=torch.int64, device=dev).repeat_interleave(C)
        self.max_reqs = S + 1
        num_slots = (S * (C // PAGE) + 1) * PAGE
        hp_rows = 1 + self.max_reqs * (P + W)
        self.layers_data = []
        for layer in range(layers):
            self.layers_data.append({
                "x": synth.make_latent(n, D, max(1, D // 100), seed=40_000 + layer, device=dev),
                "pe": synth.make_normal((n, R), 50_000 + layer, device=dev),
                "rt": synth.layer_rotation(D, layer).to(torch.bfloat16).t().contiguous().to(dev),
                "codes": torch.zeros(num_slots, D // 4, dtype=torch.uint8, device=dev),
                "params": torch.zeros(num_slots, D // 128, 2, dtype=torch.float32, device=dev),
                "rope": torch.zeros(num_slots, R, dtype=torch.bfloat16, device=dev),
                "hp": torch.zeros(hp_rows, D, dtype=torch.bfloat16, device=dev),
                "row": torch.full((num_slots,), -1, dtype=torch.int32, device=dev),
                "owner": torch.zeros(hp_rows, dtype=torch.int32, device=dev),
            })
        torch.cuda.synchronize()

    def step(self):
        from mla_kv_quant_amd import kernels, synth

        for d in self.layers_data:
            kernels.write_rows(d["x"], d["pe"], d["rt"], self.loc, self.seqs, self.positions, self.reqs,
                               d["codes"], d["params"], d["rope"], d["hp"], d["row"], d["owner"],
                               self.P, self.W, self.max_reqs, synth.DEFAULT_THRESHOLD, synth.DEFAULT_GAIN)

    def norm_step(self, rows_out: bool = True):
        """The same writes with kv_a_layernorm fused in front (x read as the
        pre-norm kv_a); with ``rows_out`` the normalized rows are also stored
        to ``y`` (the MHA prefill path's kv_b_proj input)."""
        from mla_kv_quant_amd import kernels, synth

        if not hasattr(self, "gamma"):
            self.gamma = synth.make_norm_weight(self.D, 7, device=self.dev)
            self.y = torch.empty(self.n, self.D, dtype=torch.bfloat16, device=self.dev)
        for d in self.layers_data:
            kernels.norm_write_rows(d["x"], self.gamma, 1e-6, self.y if rows_out else None, d["pe"], d["rt"], self.loc, self.seqs,
                                    self.positions, self.reqs, d["codes"], d["params"], d["rope"], d["hp"], d["row"],
                                    d["owner"], self.P, self.W, self.max_reqs, synth.DEFAULT_THRESHOLD,
                                    synth.DEFAULT_GAIN)

    def bytes_per_layer(self) -> float:
        D, R, n = self.D, self.R, self.n
        kept = self.SEQS * (self.P + self.W)
        return float(n * (2 * D + 2 * R) + n * (D // 4 + 8 * (D // 128) + 2 * R + 4) + kept * (2 * D + 4))

    def flops_per_layer(self) -> float:
        return float(2 * self.n * self.D * self.D)


# ---------------------------------------------------------------------------
# config 4b: extend (chunked prefill) over the packed prefix
# ---------------------------------------------------------------------------
class ExtendBench:
    B, TQ, PREFIX, H, D, R, P, W, PAGE = 4, 2048, 14336, 40, 256, 32, 4, 16, 64

    def __init__(self, layers: int, dev: str):
        from mla_kv_quant_amd import kernels, synth

        B, TQ, PF, H, D, R, P, W, PAGE = self.B, self.TQ, self.PREFIX, self.H, self.D, self.R, self.P, self.W, \
            self.PAGE
        self.dev = dev
        pages_per_seq = (PF + TQ) // PAGE
        perm = np.random.default_rng(2).permutation(np.arange(1, B * pages_per_seq + 1)).astype(np.int64)
        table = perm.reshape(B, pages_per_seq)
        num_slots = (B * pages_per_seq + 1) * PAGE
        # the prefix's pages (the chunk's own rows come from k_chunk)
        pp = PF // PAGE
        self.kv_indptr = torch.arange(0, B * pp + 1, pp, dtype=torch.int32, device=dev)
        self.kv_indices = torch.from_numpy(table[:, :pp].reshape(-1).astype(np.int32)).to(dev)
        self.qo_indptr = torch.arange(0, B * TQ + 1, TQ, dtype=torch.int32, device=dev)
        self.prefix = torch.full((B,), PF, dtype=torch.int64, device=dev)
        self.req = torch.arange(1, B + 1, dtype=torch.int64, device=dev)
        slots = (torch.from_numpy(table[:, :pp]).to(dev)[:, :, None] * PAGE
                 + torch.arange(PAGE, device=dev)).reshape(-1).contiguous()
        positions = torch.arange(PF, device=dev).repeat(B)
        seqs = torch.full((B * PF,), PF + TQ, dtype=torch.int64, device=dev)
        reqs = self.req.repeat_interleave(PF)
        max_reqs = B + 1
        hp_rows = 1 + max_reqs * (P + W)
        self.sm_scale = 1.0 / math.sqrt(96)
        sigma = 2.0 / (self.sm_scale * math.sqrt(D + R))
        self.layers = []
        for layer in range(layers):
            c = {
                "codes": torch.zeros(num_slots, D // 4, dtype=torch.uint8, device=dev),
                "params": torch.zeros(num_slots, D // 128, 2, dtype=torch.float32, device=dev),
                "rope": torch.zeros(num_slots, R, dtype=torch.bfloat16, device=dev),
                "hp": torch.zeros(hp_rows, D, dtype=torch.bfloat16, device=dev),
                "row": torch.full((num_slots,), -1, dtype=torch.int32, device=dev),
                "owner": torch.zeros(hp_rows, dtype=torch.int32, device=dev),
            }
            rt = synth.layer_rotation(D, layer).to(torch.bfloat16).t().contiguous().to(dev)
            x = synth.make_latent(B * PF, D, max(1, D // 100), seed=60_000 + layer, device=dev)
            pe = synth.make_normal((B * PF, R), 61_000 + layer, device=dev)
            kernels.write_rows(x, pe, rt, slots, seqs, positions, reqs, c["codes"], c["params"], c["rope"],
                               c["hp"], c["row"], c["owner"], P, W, max_reqs, synth.DEFAULT_THRESHOLD,
                               synth.DEFAULT_GAIN)
            del x, pe
            c["q"] = synth.make_normal((B * TQ, H, D + R), 62_000 + layer, std=sigma, device=dev)
            c["kc"] = torch.cat([synth.make_latent(B * TQ, D, 3, seed=63_000 + layer, device=dev),
                                 synth.make_normal((B * TQ, R), 64_000 + layer, device=dev)], 1).contiguous()
            self.layers.append(c)
        self.out = torch.empty(B * TQ, H, D, dtype=torch.bfloat16, device=dev)
        # key rows gathered per call (one layer at a time: one workspace serves all layers)
        self.key_rows = B * (PF + TQ)
        self.ws = torch.empty(self.key_rows, D + R, dtype=torch.float16, device=dev)
        torch.cuda.synchronize()

    def step(self):
        from mla_kv_quant_amd import kernels

        for c in self.layers:
            kernels.extend_fwd(c["q"], c["kc"], self.qo_indptr, self.kv_indptr, self.kv_indices, self.prefix,
                               self.req, c["codes"], c["params"], c["rope"], c["hp"], self.TQ, self.out,
                               self.sm_scale, self.P, self.W, self.PAGE, workspace=self.ws, key_rows=self.key_rows)

    def flops_per_layer(self) -> float:
        """Algorithmic flops: 2 H (2 D + R) per (query, visible key) pair."""
        B, TQ, PF, H, D, R = self.B, self.TQ, self.PREFIX, self.H, self.D, self.R
        pairs = B * (TQ * PF + TQ * (TQ + 1) // 2)
        return float(2 * H * (2 * D + R) * pairs)


def extend_result(args, dev: str, layers: int = 2) -> dict:
    eb = ExtendBench(layers, dev)
    ms = time_loop(eb.step, max(2, args.steps // 4), 1)
    ms_layer = ms / layers
    tflops = eb.flops_per_layer() / (ms_layer * 1e-3) / 1e12
    res = {
        "workload": "cfg4b extend: batch 4 x 2048 causal queries over a 14336-token INT2 prefix + s4r16 window, "
                    "40 heads, latent 256, rope 32, page 64",
        "ms_per_layer": round(ms_layer, 4),
        "tflops": round(tflops, 1),
        "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
    }
    print(f"[bench] extend: {ms_layer:.3f} ms/layer, {tflops:.0f} TFLOP/s", file=sys.stderr, flush=True)
    del eb
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------
# CPU baseline (oracle on the host cores)
# ---------------------------------------------------------------------------
def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_runs(fn, runs: int = 5):
    """1 warm-up, then ``runs`` timed calls; returns (median s, all s)."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), ts


def _pool_np(c: dict) -> dict:
    return {
        "codes": c["codes"].cpu().numpy(),
        "params": c["params"].cpu().numpy(),
        "rope": c["rope"].cpu().view(torch.int16).numpy().view(np.uint16),
        "hp": c["hp"].cpu().view(torch.int16).numpy().view(np.uint16),
    }


def _attention_leg(db: "DecodeBench", seqs: int, batch: int):
    """One layer of the oracle's dequantize-then-attention (torch CPU, FP32) over
    ``seqs`` sequences of ``db``'s layer 0, scaled to ``batch`` sequences."""
    from oracle import attention

    c = db.caches[0]
    pool = _pool_np(c)
    pt = db.kv_indices.cpu().numpy().reshape(db.B, -1)
    q = c["q"].cpu()
    D = db.D
    slots = [(pt[b][:, None] * db.PAGE + np.arange(db.PAGE)).reshape(-1) for b in range(seqs)]
    lens = [int(v) for v in db.lengths[:seqs]]
    med, ts = _median_runs(lambda: attention.decode(pool, q[:seqs, :, :D], q[:seqs, :, D:], slots, lens,
                                                    list(range(1, seqs + 1)), db.P, db.W, db.sm_scale, D, "fp32"))
    scale = batch / seqs
    return {"value": round(med * scale * 1e6, 1), "unit": "us/layer", "median_s_sample": round(med, 4),
            "runs_s": [round(t, 4) for t in ts], "sample": f"{seqs} of {batch} sequences, scaled x{scale:g}"}


def cpu_baseline(db: "DecodeBench", dev: str):
    """The reference arithmetic restated in PyTorch on the host cores (the
    oracle): cfg0 codec + QDQ, one cfg1 layer of FP32 rotation GEMM + QDQ, and
    one layer of dequantize-then-attention at cfg2 and cfg4a. Median of 5 runs
    after one warm-up each, on bounded samples scaled to the full workload."""
    from oracle import codec
    from mla_kv_quant_amd import synth

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    legs = {}
    # cfg0: codec + QDQ on [4096, 512] (rotated rows, oscar.py:120-144 / quantizer.py:102-124)
    rot = synth.make_rotation(512, 90)
    x0 = synth.make_latent(4096, 512, 8, seed=90)
    med, ts = _median_runs(lambda: codec.rotate_quantize(x0, rot))
    legs["cfg0_codec_qdq"] = {"value": round(med * 1e3, 2), "unit": "ms", "rows": 4096,
                              "runs_s": [round(t, 4) for t in ts]}
    # cfg1: one layer = FP32 rotation GEMM + QDQ of all 131072 rows
    x1 = synth.make_latent(131072, 512, 5, seed=91)
    med, ts = _median_runs(lambda: codec.rotate_quantize(x1, rot))
    legs["cfg1_rotate_qdq_layer"] = {"value": round(med * 1e3, 1), "unit": "ms/layer",
                                     "sample": "all 131072 rows of one layer", "runs_s": [round(t, 4) for t in ts]}
    # cfg2 / cfg4a: one layer of dequantize-then-attention (cfg2 whole, cfg4a a quarter of the batch)
    legs["cfg2_attention_layer"] = _attention_leg(db, db.B, db.B)
    db4 = DecodeBench(1, dev, B=16, lengths=[16384] * 16, H=40, D=256, R=32, seed=4)
    legs["cfg4a_attention_layer"] = _attention_leg(db4, 16, 64)
    del db4
    torch.cuda.empty_cache()
    head = legs["cfg2_attention_layer"]
    return {"value": head["value"], "unit": "us/layer", "cores": threads, "kind": "port",
            "sample": f"cfg2 leg: oracle dequantize-then-attention (torch CPU, FP32) over all {db.B} sequences x "
                      f"{db.L} tokens of one layer, median of 5 runs after one warm-up (about 8 s of CPU work "
                      f"with the other legs)",
            "nproc": threads, "cpu_model": _cpu_model(), "legs": legs}


def read_traffic():
    """HBM bytes per decode_stage1 dispatch from the committed rocprofv3 summary, if any."""
    f = ROOT / "profiles" / "decode_cfg2_traffic.json"
    if f.exists():
        try:
            return json.loads(f.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            return None
    return None


def read_probe(nbytes: int = 4 << 30, reps: int = 10) -> float:
    """Achievable HBM read rate: GB/s over ``nbytes`` read once and reduced to
    a few bytes (a read-only stream like decode's), the better of torch's sum
    over fp32 and a bf16 matrix-vector product (rocBLAS GEMV)."""
    x = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    ms_sum = time_loop(lambda: x.sum(), reps, 2)
    a = x.view(torch.bfloat16).view(-1, 8192)
    v = torch.ones(8192, dtype=torch.bfloat16, device="cuda")
    ms_mv = time_loop(lambda: torch.mv(a, v), reps, 2)
    del x, a
    torch.cuda.empty_cache()
    return nbytes / (min(ms_sum, ms_mv) * 1e-3) / 1e9


def copy_probe(nbytes: int = 1 << 30, reps: int = 10) -> float:
    """Achievable HBM rate: GB/s (read + write) of a device-to-device copy of ``nbytes``."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    ms = time_loop(lambda: dst.copy_(src), reps, 2)
    del src, dst
    torch.cuda.empty_cache()
    return 2.0 * nbytes / (ms * 1e-3) / 1e9


def reported_decode_result(args, dev: str, name: str) -> dict:
    """Decode at the library's own split policy (the reference's 129 splits requested,
    capped by the library at one working block per CU): cfg3 (ragged large batch) and
    cfg4a (MiniCPM3 shape), 4 layers with their own buffers; "serve_b8" / "serve_b16":
    DeepSeek-V2-Lite shape at the reference's serving batch sizes (serve.py:157-158,164),
    8 layers."""
    from mla_kv_quant_amd import kernels

    layers = 4
    if name == "cfg3":
        lens = np.random.default_rng(3).integers(2048, 8193, size=128)
        db = DecodeBench(layers, dev, B=128, lengths=lens, H=16, D=512, R=64, seed=3)
        workload = "cfg3 decode: batch 128, ragged context U[2048,8192], 16 heads, latent 512, rope 64, page 64 shuffled"
    elif name == "cfg4a":
        db = DecodeBench(layers, dev, B=64, lengths=[16384] * 64, H=40, D=256, R=32, seed=4)
        workload = "cfg4a decode: batch 64 x context 16384, 40 heads, latent 256, rope 32, page 64 shuffled"
    else:
        B = int(name[len("serve_b"):])
        layers = 8
        db = DecodeBench(layers, dev, B=B, seed=5 + B)
        workload = (f"serving decode: batch {B} x context 16384, 16 heads, latent 512, rope 64, page 64 shuffled "
                    f"(the reference's graph batch sizes, serve.py:157-158,164)")
    db.alloc_scratch(129)
    db.set_splits(129)  # the reference's static split count (serve.py:121,163,198)
    ns = kernels.decode_split_cap(db.B, db.H, db.D, 129)
    steps = max(5, args.steps // 2)
    time_loop(db.step, steps, args.warmup)  # a first pass over fresh buffers runs slower: not timed
    ms = float(np.median([time_loop(db.step, steps, 1) for _ in range(3)]))
    us = ms * 1000.0 / layers
    # stage 1 alone (decode_partials honours the count and launches max_kv_splits + 1
    # split rows) at the count the fused call used, with scratch sized to it
    db.alloc_scratch(ns)
    db.set_splits(ns)
    ms1 = float(np.median([time_loop(db.step_partials, steps, 1) for _ in range(3)]))
    us1 = ms1 * 1000.0 / layers
    ach1 = db.bytes_per_layer(with_out=False) / (us1 * 1e-6) / 1e9
    res = {
        "workload": workload,
        "us_per_layer": round(us, 3),
        "hbm_frac_layer": round(db.bytes_per_layer() / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "stage1_us": round(us1, 3),
        "stage1_gbs": round(ach1, 1),
        "stage1_hbm_frac": round(ach1 / HBM_PEAK_GBS, 4),
        "mfma_frac": round(db.flops_per_layer() / (us1 * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "num_kv_splits_requested": 129,
        "num_kv_splits_used": ns,
        "tokens": int(db.lengths.sum()),
    }
    print(f"[bench] {name}: {us:.2f} us/layer, stage 1 {us1:.2f} us ({ach1:.0f} GB/s)", file=sys.stderr, flush=True)
    del db
    torch.cuda.empty_cache()
    return res


def qdq_result(args, dev: str) -> dict:
    """GPU rotate_quantize (the fake-quantized cache path) on 32 x 4096 rows of D = 512."""
    from mla_kv_quant_amd import qdq, synth

    n, D = 32 * 4096, 512
    x = synth.make_latent(n, D, 5, seed=70_000, device=dev).reshape(32, 4096, D)
    rot = synth.make_rotation(D, 70)
    ms = time_loop(lambda: qdq.rotate_quantize(x, rot), max(5, args.steps // 2), args.warmup)
    res = {"workload": "rotate_quantize (QDQ) of 32 x 4096 latent rows, D=512, two launches + scratch",
           "rows": n, "us": round(ms * 1000, 2), "mrows_per_s": round(n / (ms * 1e-3) / 1e6, 1)}
    print(f"[bench] qdq: {ms * 1000:.1f} us for {n} rows", file=sys.stderr, flush=True)
    del x
    torch.cuda.empty_cache()
    return res


def writer_result(args, dev: str) -> dict:
    wb = WriterBench(args.layers, dev)
    wms = time_loop(wb.step, max(3, args.steps // 2), args.warmup)
    wus = wms * 1000.0 / args.layers
    wach = wb.bytes_per_layer() / (wus * 1e-6) / 1e9
    res = {
        "workload": "cfg1 writer: 64 seqs x 2048-token prefill chunk, 27 layers with own buffers",
        "mtokens_per_s": round(wb.n * args.layers / (wms * 1e-3) / 1e6, 1),
        "us_per_layer": round(wus, 3),
        "hbm_achieved_gbs": round(wach, 1),
        "hbm_frac": round(wach / HBM_PEAK_GBS, 4),
        "mfma_frac": round(wb.flops_per_layer() / (wus * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
    }
    # dequantize-rows of the cache just written (MHA prefill over a quantized
    # prefix): every cfg1 row of one layer, rotated frame and rotated back
    from mla_kv_quant_amd import kernels

    d0 = wb.layers_data[0]
    r_eff = d0["rt"].t().contiguous()
    rows = torch.empty(wb.n, wb.D + wb.R, dtype=torch.bfloat16, device=dev)
    for key, rot in (("assemble_us", None), ("assemble_unrotate_us", r_eff)):
        ams = time_loop(lambda: kernels.assemble_rows(wb.loc, d0["codes"], d0["params"], d0["rope"], d0["hp"],
                                                      d0["row"], d0["owner"], rot, rows),
                        max(5, args.steps), args.warmup)
        res[key] = round(ams * 1000.0, 3)
    del rows
    for key, rows_out in (("norm_fused_us_per_layer", False), ("norm_fused_rows_out_us_per_layer", True)):
        nms = time_loop(lambda: wb.norm_step(rows_out), max(3, args.steps // 2), args.warmup)
        res[key] = round(nms * 1000.0 / args.layers, 3)
    print(f"[bench] writer: {wus:.2f} us/layer, {res['mtokens_per_s']} Mtok/s; with kv_a_layernorm fused: "
          f"{res['norm_fused_us_per_layer']} us/layer, and the normalized rows stored: "
          f"{res['norm_fused_rows_out_us_per_layer']} us/layer; dequantize rows {res['assemble_us']} us, rotated "
          f"back {res['assemble_unrotate_us']} us", file=sys.stderr, flush=True)
    del wb
    torch.cuda.empty_cache()
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the packed-INT2 path is single-GPU here); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        sys.exit(2)
    dev = "cuda:0"
    torch.cuda.set_device(0)
    if args.copy_probe:
        print(json.dumps({"copy_gbs": round(copy_probe(), 1), "bytes": 1 << 30}), flush=True)
        return
    if args.read_probe:
        print(json.dumps({"read_gbs": round(read_probe(), 1), "bytes": 4 << 30}), flush=True)
        return
    from mla_kv_quant_amd import _lib

    _lib.load()
    if args.writer_only:
        print(json.dumps(writer_result(args, dev)), flush=True)
        return
    if args.extend_only:
        print(json.dumps(extend_result(args, dev)), flush=True)
        return
    if args.reported_only:
        out = {k: reported_decode_result(args, dev, k) for k in ("cfg3", "cfg4a", "serve_b8", "serve_b16")}
        out["qdq"] = qdq_result(args, dev)
        print(json.dumps(out), flush=True)
        return
    t_setup = time.time()
    db = DecodeBench(args.layers, dev)
    print(f"[bench] decode caches written for {args.layers} layers in {time.time() - t_setup:.1f}s", file=sys.stderr,
          flush=True)
    # split policy: one working block per CU (num_kv_splits = ceil(CUs / B) INT2
    # splits + the window split), fixed before timing; --splits overrides it.
    # The reference's static 129 (serve.py:198) is timed beside it.
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    ns_best = args.splits if args.splits else -(-cus // db.B) + 1
    # the two settings alternate over three rounds (medians), both warmed
    # first, so that neither carries the other's warm-up or the cold caches
    # of the first timed loop
    def at(ns, steps):
        db.alloc_scratch(ns)
        db.set_splits(ns)
        return time_loop(db.step, steps, args.warmup)

    at(129, 1)
    at(ns_best, 1)
    r129, rbest = [], []
    for _ in range(3):
        r129.append(at(129, max(3, args.steps // 2)))
        rbest.append(at(ns_best, args.steps))
    ms129, ms = statistics.median(r129), statistics.median(rbest)
    us_layer = ms * 1000.0 / args.layers
    print(f"[bench] decode: {ns_best} splits {us_layer:.2f} us/layer, the reference's 129 splits "
          f"{ms129 * 1000.0 / args.layers:.2f} us/layer", file=sys.stderr, flush=True)
    bpl = db.bytes_per_layer()
    # the dominant kernel (stage 1) timed alone: same events, same stream, one launch per layer
    ms1 = time_loop(db.step_partials, args.steps, args.warmup)
    us_stage1 = ms1 * 1000.0 / args.layers
    b1 = db.bytes_per_layer(with_out=False)
    achieved = b1 / (us_stage1 * 1e-6) / 1e9
    copy_gbs = copy_probe()
    read_gbs = read_probe()
    print(f"[bench] decode: {us_layer:.2f} us/layer; stage 1 {us_stage1:.2f} us/launch, {achieved:.0f} GB/s "
          f"(device copy {copy_gbs:.0f} GB/s)", file=sys.stderr, flush=True)

    result = {
        "metric": "INT2 MLA decode attn us/layer (cfg2: B=32 x 16K, H=16, D=512, R=64)",
        "value": round(us_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int2-cache/fp16-mfma(latent)+bf16-mfma(rope)/fp32-acc",
        "data": "synthetic (seeded N(0,1) latents, 1% outlier channels x20, seeded orthogonal rotations)",
        "config": {"workload": "cfg2 decode: batch 32 x context 16384, 16 heads, latent 512, rope 64, "
                               "s4r16 window, page 64 shuffled, 27 layers with own buffers",
                   "batch": db.B, "context": db.L, "heads": db.H, "layers": args.layers,
                   "num_kv_splits": ns_best, "split_policy": "ceil(CUs / B) + 1 (the library's cap)",
                   "us_per_layer_at_129_splits": round(ms129 * 1000.0 / args.layers, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "kernel": "decode_stage1<512,64,1>", "us_per_launch": round(us_stage1, 3),
                     "algorithmic_bytes_per_launch": b1,
                     "layer_frac": round(bpl / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "copy_gbs": round(copy_gbs, 1),
                     "read_gbs": round(read_gbs, 1),
                     "frac_of_read": round(achieved / read_gbs, 4),
                     "frac_of_copy": round(achieved / copy_gbs, 4),
                     "mfma_frac": round(db.flops_per_layer() / (us_stage1 * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)},
    }
    if not args.no_writer or not args.no_extend or not args.no_reported:
        del db.caches
        torch.cuda.empty_cache()
    if not args.no_writer:
        result["writer"] = writer_result(args, dev)
    if not args.no_extend:
        result["extend"] = extend_result(args, dev)
    if not args.no_reported:
        result["reported"] = {k: reported_decode_result(args, dev, k)
                              for k in ("cfg3", "cfg4a", "serve_b8", "serve_b16")}
        result["reported"]["qdq"] = qdq_result(args, dev)
    if not args.no_cpu:
        if not hasattr(db, "caches"):
            db = DecodeBench(1, dev)
        result["cpu_baseline"] = cpu_baseline(db, dev)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
