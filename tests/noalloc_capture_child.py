"""Child process of tests/test_zz_no_alloc.py: the allocation-free decode's
first call in a fresh process made under HIP graph capture (so its one-time
scratch address lookup runs while the stream is capturing), then the graph
replayed with eager work in between; every replay must equal rolaq_decode_fwd
bit for bit. Exits 0 on success."""

import math
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402
import torch  # noqa: E402

from mla_kv_quant_amd import _lib, kernels  # noqa: E402
from mla_kv_quant_amd.kernels import _p, _stream  # noqa: E402
from tests.helpers import build_pool, index_lists, make_queries, pool_to_gpu  # noqa: E402


def main() -> int:
    dev = "cuda"
    D, R, H, P, W, page = 512, 64, 16, 4, 16, 64
    lengths = [300, 1025, 64]
    splits = [3, 5, 2]
    sm = 1.0 / math.sqrt(192)
    pool, slots, pages, reqs, _ = build_pool(lengths, D, R, P, W, page, seed=29)
    gp = pool_to_gpu(pool)
    q = make_queries(len(lengths), H, D, R, sm, seed=30).to(dev)
    indptr, indices = index_lists(slots, pages, page)
    seq = torch.tensor(lengths, dtype=torch.int64, device=dev)
    req = torch.tensor(np.asarray(reqs), dtype=torch.int64, device=dev)
    ns = torch.tensor(splits, dtype=torch.int32, device=dev)
    B, max_splits, max_reqs = len(lengths), 8, len(lengths) + 1
    logits = torch.empty(B, H, max_splits + 1, D, device=dev)
    lse = torch.empty(B, H, max_splits + 1, device=dev)
    ref = torch.empty(B, H, D, dtype=torch.bfloat16, device=dev)
    kernels.decode_fwd(q, gp["codes"], gp["params"], gp["rope"], gp["hp"], indptr, indices, seq, req, ns,
                       max_splits, logits, lse, ref, sm, P, W, page, max_reqs=max_reqs)
    torch.cuda.synchronize()
    out = torch.full((B, H, D), float("nan"), dtype=torch.bfloat16, device=dev)
    lib = _lib.load()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream), torch.cuda.graph(graph, stream=stream):
        rc = lib.rolaq_decode_fwd_noalloc(
            _p(q), q.stride(0), q.stride(1), _p(gp["codes"]), _p(gp["params"]), _p(gp["rope"]), _p(gp["hp"]),
            _p(indptr), _p(indices), page, _p(seq), _p(req), max_reqs, _p(ns), max_splits, B, H, D, R, P, W, sm,
            _p(out), out.stride(0), out.stride(1), _stream(q))
    if rc != 0:
        print("first call under capture failed:", lib.rolaq_last_error().decode(), flush=True)
        return 1
    for k in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(out, ref):
            print(f"replay {k} differs from rolaq_decode_fwd", flush=True)
            return 1
        _ = (q.float() * 2).sum().item()  # eager work between replays
    print("ok: first call under capture, 3 replays equal rolaq_decode_fwd", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
