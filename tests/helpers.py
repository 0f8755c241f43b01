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
