"""GPU: the allocation-free decode entry point against rolaq_decode_fwd.

rolaq_decode_fwd_noalloc runs the same kernels as rolaq_decode_fwd with the
split partials in the library's static per-GPU scratch array instead of the
caller's attn_logits / attn_lse, so its output must equal rolaq_decode_fwd's
bit for bit. Two calls in a row, the second with a smaller batch and fewer
splits (the array keeps the first call's partials), then a request whose
workspace exceeds the array, which must be rejected before any launch.
"""

import math

import numpy as np
import pytest
import torch

from mla_kv_quant_amd import _lib, kernels
from mla_kv_quant_amd.kernels import _p, _stream
from tests.helpers import build_pool, index_lists, make_queries, pool_to_gpu

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _noalloc(gp, q, indptr, indices, page, seq, req, ns, max_splits, P, W, sm_scale, max_reqs, out):
    B, H, _ = q.shape
    D = gp["codes"].shape[1] * 4
    R = q.shape[2] - D
    return _lib.load().rolaq_decode_fwd_noalloc(
        _p(q), q.stride(0), q.stride(1), _p(gp["codes"]), _p(gp["params"]), _p(gp["rope"]), _p(gp["hp"]),
        _p(indptr), _p(indices), int(page), _p(seq), _p(req), int(max_reqs), _p(ns), int(max_splits), B, H, D, R,
        int(P), int(W), float(sm_scale), _p(out), out.stride(0), out.stride(1), _stream(q))


def _both(gp, q, slots, pages, lengths, reqs, page, splits, max_splits, P, W, sm_scale, max_reqs):
    B, H, _ = q.shape
    D = gp["codes"].shape[1] * 4
    indptr, indices = index_lists(slots, pages, page)
    seq = torch.tensor(lengths, dtype=torch.int64, device=DEV)
    req = torch.tensor(np.asarray(reqs), dtype=torch.int64, device=DEV)
    ns = torch.tensor(splits, dtype=torch.int32, device=DEV)
    qd = q.to(DEV)
    logits = torch.empty(B, H, max_splits + 1, D, device=DEV)
    lse = torch.empty(B, H, max_splits + 1, device=DEV)
    ref = torch.empty(B, H, D, dtype=torch.bfloat16, device=DEV)
    kernels.decode_fwd(qd, gp["codes"], gp["params"], gp["rope"], gp["hp"], indptr, indices, seq, req, ns,
                       max_splits, logits, lse, ref, sm_scale, P, W, page, max_reqs=max_reqs)
    out = torch.full((B, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    _lib.check(_noalloc(gp, qd, indptr, indices, page, seq, req, ns, max_splits, P, W, sm_scale, max_reqs, out))
    torch.cuda.synchronize()
    return out.cpu(), ref.cpu()


@pytest.mark.parametrize("D,R,H,page", [(512, 64, 16, 64), (256, 32, 40, 16)])
def test_noalloc_decode_equals_decode_fwd(D, R, H, page):
    P, W = 4, 16
    sm_scale = 1.0 / math.sqrt(192 if D == 512 else 96)
    lengths = [5, 700, 2049, 130, 64 * 9, 1500]
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, page, seed=23)
    gp = pool_to_gpu(pool)
    max_reqs = len(lengths) + 1
    q = make_queries(len(lengths), H, D, R, sm_scale, seed=7)
    # first call: six requests, up to 17 splits
    out, ref = _both(gp, q, slots, pages, lengths, reqs, page, [2, 5, 17, 3, 9, 4], 17, P, W, sm_scale, max_reqs)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    # second call: a smaller batch with fewer splits over the same scratch
    sub = [1, 3, 4]
    out2, ref2 = _both(gp, q[sub].contiguous(), [slots[i] for i in sub], [pages[i] for i in sub],
                       [lengths[i] for i in sub], [reqs[i] for i in sub], page, [3, 2, 5], 5, P, W, sm_scale,
                       max_reqs)
    assert torch.equal(out2.view(torch.int16), ref2.view(torch.int16))
    assert torch.isfinite(out2.float()).all()


def test_noalloc_rejects_oversized_workspace():
    D, R, H, B, max_splits = 512, 64, 128, 64, 129  # 64*128*130*513*4 bytes >> 32 MiB
    q = torch.zeros(B, H, D + R, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(B, H, D, dtype=torch.bfloat16, device=DEV)
    z = torch.zeros(16, dtype=torch.int64, device=DEV)
    rc = _lib.load().rolaq_decode_fwd_noalloc(
        _p(q), q.stride(0), q.stride(1), _p(z), _p(z), _p(z), _p(z), _p(z), _p(z), 1, _p(z), _p(z), 1, _p(z),
        max_splits, B, H, D, R, 4, 16, 0.1, _p(out), out.stride(0), out.stride(1), _stream(q))
    assert rc == _lib.ROLAQ_ERR_INVALID
    assert "static scratch" in _lib.load().rolaq_last_error().decode()


def test_noalloc_captured_replays_equal_decode_fwd():
    """Captured in a HIP graph after eager calls (its scratch address already
    looked up), then replayed three times with eager work in between: every
    replay equals rolaq_decode_fwd bit for bit, and so does a second graph
    over a smaller batch sharing the same static scratch."""
    D, R, H, P, W, page = 256, 32, 40, 4, 16, 16
    sm = 1.0 / math.sqrt(96)
    lengths = [700, 33, 1500]
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, page, seed=31)
    gp = pool_to_gpu(pool)
    q = make_queries(len(lengths), H, D, R, sm, seed=32).to(DEV)
    max_reqs = len(lengths) + 1
    for sel, splits, max_splits in (([0, 1, 2], [4, 2, 6], 8), ([2], [3], 4)):
        qs = q[sel].contiguous()
        s_slots, s_pages = [slots[i] for i in sel], [pages[i] for i in sel]
        s_len, s_req = [lengths[i] for i in sel], [reqs[i] for i in sel]
        out_e, ref = _both(gp, qs, s_slots, s_pages, s_len, s_req, page, splits, max_splits, P, W, sm, max_reqs)
        assert torch.equal(out_e, ref)
        indptr, indices = index_lists(s_slots, s_pages, page)
        seq = torch.tensor(s_len, dtype=torch.int64, device=DEV)
        req = torch.tensor(np.asarray(s_req), dtype=torch.int64, device=DEV)
        ns = torch.tensor(splits, dtype=torch.int32, device=DEV)
        out = torch.full((len(sel), H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
        graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream), torch.cuda.graph(graph, stream=stream):
            rc = _noalloc(gp, qs, indptr, indices, page, seq, req, ns, max_splits, P, W, sm, max_reqs, out)
        _lib.check(rc)
        for _ in range(3):
            out.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out.cpu(), ref)
            _ = (qs.float() * 2).sum().item()  # eager work between replays


def test_noalloc_first_call_under_capture():
    """In a fresh process, the entry point's first call (which looks up the
    static scratch's device address once) made under graph capture: the
    capture succeeds and its replays equal rolaq_decode_fwd bit for bit
    (tests/noalloc_capture_child.py, started as a child process)."""
    import subprocess
    import sys
    from pathlib import Path

    child = Path(__file__).resolve().parent / "noalloc_capture_child.py"
    res = subprocess.run([sys.executable, "-u", str(child)], capture_output=True, text=True, timeout=240)
    print(res.stdout[-2000:], res.stderr[-2000:])
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-2000:]
