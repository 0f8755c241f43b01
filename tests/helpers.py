"""Shared builders for the parity tests: oracle-written pools, GPU copies, queries."""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import window
from mla_kv_quant_amd import synth


def alloc_slots(lengths, page: int, seed: int, spare_pages: int = 3):
    """Shuffled physical pages (slot 0's page is never used); returns
    (per-sequence slot arrays, per-sequence page lists, num_slots)."""
    npages = [int(math.ceil(L / page)) if L > 0 else 0 for L in lengths]
    total = sum(npages) + spare_pages
    perm = np.random.default_rng(seed).permutation(np.arange(1, total + 1))
    slots, pages, k = [], [], 0
    for L, n in zip(lengths, npages):
        pg = perm[k:k + n]
        k += n
        pages.append(pg)
        s = (pg[:, None] * page + np.arange(page)[None, :]).reshape(-1)[:L]
        slots.append(s.astype(np.int64))
    return slots, pages, (total + 1) * page


def build_pool(lengths, D, R, P, W, page, seed, max_reqs=None, threshold=0.9810652732849121,
               gain=1.16, outliers=None):
    """Oracle pool holding ``len(lengths)`` sequences written as prefills."""
    B = len(lengths)
    max_reqs = max_reqs or B + 1
    slots, pages, num_slots = alloc_slots(lengths, page, seed)
    pool = window.new_pool(num_slots, D, R, max_reqs, P, W)
    rot = synth.make_rotation(D, seed + 17)
    reqs = np.arange(B) + 1  # request 0 unused
    for b, L in enumerate(lengths):
        if L == 0:
            continue
        x = synth.make_latent(L, D, outliers if outliers is not None else max(1, D // 100), seed=seed * 31 + b)
        pe = synth.make_normal((L, R), seed * 37 + b)
        window.write_rows(pool, x, pe, slots[b], np.full(L, L), np.full(L, reqs[b]), rot, threshold, gain,
                          P, W, max_reqs, positions=np.arange(L))
    return pool, slots, pages, reqs, rot


def pool_to_gpu(pool: dict, device="cuda"):
    return {
        "codes": torch.from_numpy(pool["codes"]).to(device),
        "params": torch.from_numpy(pool["params"]).to(device),
        "rope": torch.from_numpy(pool["rope"].view(np.int16)).view(torch.bfloat16).to(device),
        "hp": torch.from_numpy(pool["hp"].view(np.int16)).view(torch.bfloat16).to(device),
        "row_of_slot": torch.from_numpy(pool["row_of_slot"]).to(device),
        "owner_of_row": torch.from_numpy(pool["owner_of_row"]).to(device),
    }


def index_lists(slots, pages, page_size: int, device="cuda"):
    """SGLang-style kv_indptr/kv_indices (token slots for page_size 1, pages otherwise)."""
    if page_size == 1:
        lists = slots
    else:
        lists = pages
    indptr = np.zeros(len(lists) + 1, np.int32)
    indptr[1:] = np.cumsum([len(x) for x in lists])
    flat = np.concatenate([np.asarray(x, np.int32) for x in lists]) if indptr[-1] else np.zeros(1, np.int32)
    return torch.from_numpy(indptr).to(device), torch.from_numpy(flat).to(device)


def make_queries(B, H, D, R, sm_scale, seed, logit_std=2.0):
    sigma = logit_std / (sm_scale * math.sqrt(D + R))
    q = synth.make_normal((B, H, D + R), seed, std=sigma)
    return q


def bf16_np_to_torch(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def gpu_pool_to_oracle(gp: dict) -> dict:
    """Host copy of a GPU pool in the oracle's dict format (bf16 as uint16 bits)."""
    def bits(t):
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    return {
        "codes": gp["codes"].cpu().numpy(),
        "params": gp["params"].cpu().numpy(),
        "rope": bits(gp["rope"]),
        "hp": bits(gp["hp"]),
        "row_of_slot": gp["row_of_slot"].cpu().numpy(),
        "owner_of_row": gp["owner_of_row"].cpu().numpy(),
    }


def gpu_written_pool(lengths, D, R, P, W, page, seed, max_reqs=None, reqs=None, outliers=None,
                     device="cuda"):
    """A pool holding ``len(lengths)`` sequences written as prefills by the
    library's fused writer (used for sizes where the CPU oracle writer is too
    slow; the writer itself is held to the oracle in test_gpu_writer.py).
    Returns (gpu dict, slots per sequence, pages per sequence, request indices)."""
    from mla_kv_quant_amd import kernels

    B = len(lengths)
    max_reqs = max_reqs or B + 1
    reqs = np.asarray(reqs if reqs is not None else np.arange(B) + 1, dtype=np.int64)
    slots, pages, num_slots = alloc_slots(lengths, page, seed)
    hp_rows = 1 + max_reqs * (P + W)
    gp = {
        "codes": torch.zeros(num_slots, D // 4, dtype=torch.uint8, device=device),
        "params": torch.zeros(num_slots, D // 128, 2, dtype=torch.float32, device=device),
        "rope": torch.zeros(num_slots, R, dtype=torch.bfloat16, device=device),
        "hp": torch.zeros(hp_rows, D, dtype=torch.bfloat16, device=device),
        "row_of_slot": torch.full((num_slots,), -1, dtype=torch.int32, device=device),
        "owner_of_row": torch.zeros(hp_rows, dtype=torch.int32, device=device),
    }
    rt = synth.make_rotation(D, seed + 17).to(torch.bfloat16).t().contiguous().to(device)
    live = [b for b in range(B) if lengths[b] > 0]
    n = int(sum(lengths))
    if n:
        loc = torch.from_numpy(np.concatenate([slots[b] for b in live])).to(device)
        pos = torch.from_numpy(np.concatenate([np.arange(lengths[b]) for b in live])).to(device)
        seq = torch.from_numpy(np.concatenate([np.full(lengths[b], lengths[b]) for b in live])).to(device)
        rq = torch.from_numpy(np.concatenate([np.full(lengths[b], reqs[b]) for b in live])).to(device)
        x = synth.make_latent(n, D, outliers if outliers is not None else max(1, D // 100), seed=seed * 31,
                              device=device)
        pe = synth.make_normal((n, R), seed * 37, device=device)
        kernels.write_rows(x, pe, rt, loc, seq, pos, rq, gp["codes"], gp["params"], gp["rope"], gp["hp"],
                           gp["row_of_slot"], gp["owner_of_row"], P, W, max_reqs, 0.9810652732849121, 1.16)
        torch.cuda.synchronize()
    return gp, slots, pages, reqs


def fused_splits(splits, H, D, max_splits):
    """The split counts rolaq_decode_fwd uses for a batch that requests
    ``splits``: each capped at the library's split cap for (B, H, D) on the
    current device (whose partials the fused call writes)."""
    from mla_kv_quant_amd import kernels
    cap = kernels.decode_split_cap(len(splits), H, D, max_splits)
    return [min(int(ns), cap) for ns in splits]


def fused_partials(logits, lse, B, H, D, max_splits):
    """The split partials a fused rolaq_decode_fwd call left in its scratch,
    in the standard ``[B, H, max_splits + 1, D]`` / ``[B, H, max_splits + 1]``
    shape (slots past the fused call's stride are NaN). The fused call stores
    them from the start of the buffers at a stride of S1c = min(cap - 1,
    max_splits) + 1 slots per (sequence, head)."""
    import torch
    from mla_kv_quant_amd import kernels
    cap = kernels.decode_split_cap(B, H, D, max_splits)
    s1c = max(min(cap - 1, max_splits), 1) + 1
    n = B * H * s1c
    lg = torch.full((B, H, max_splits + 1, D), float("nan"), dtype=logits.dtype, device=logits.device)
    ls = torch.full((B, H, max_splits + 1), float("nan"), dtype=lse.dtype, device=lse.device)
    lg[:, :, :s1c] = logits.reshape(-1)[: n * D].view(B, H, s1c, D)
    ls[:, :, :s1c] = lse.reshape(-1)[:n].view(B, H, s1c)
    return lg, ls


def rotated_latent(n, D, outliers, seed, rotation):
    """bf16 ``[n, D]`` latent rows in a layer's rotated frame: synthetic rows
    (N(0,1), ``outliers`` channels x20) times ``R_eff = fp32(bf16(R))``, the
    frame the cache stores and the extend reader's chunk keys live in
    (mla_quant/quantizer.py:117-118)."""
    x = synth.make_latent(n, D, outliers, seed=seed).float()
    return (x @ rotation.to(torch.bfloat16).float()).to(torch.bfloat16)
