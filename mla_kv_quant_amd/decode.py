"""Drop-in decode reader entry points (reference interface, HIP implementation).

``prepare_gf_splits`` mirrors deployment/patches/rolaq_sglang.patch:81-92 and
``packed_mla_decode_gf_fwd`` the packed decode reader its call site drives
(rolaq_sglang.patch:51-111): stage 1 over ``max(ns - 1, 1)`` splits plus the
window split slot, LSE merge, output in the rotated latent frame. The rows it
attends over are the reference's stored rows (INT2 rows dequantized and
rounded to bf16, mla_quant/quantizer.py:120; BF16 window rows).
"""

from __future__ import annotations

import torch

from . import kernels

prepare_gf_splits = kernels.prepare_gf_splits


def packed_mla_decode_gf_fwd(q, o, pool, layer_id, kv_indptr, kv_indices, num_kv_splits, max_kv_splits,
                             attn_logits, attn_lse, sm_scale, seq_lens=None, req_pool_indices=None,
                             page_size: int = 1, has_hp: bool = True):
    """Absorbed MLA decode over layer ``layer_id`` of ``pool``.

    ``q``: bf16 ``[B, H, D + R]`` (absorbed latent query | rope query), ``o``:
    bf16 ``[B, H, D]``. ``kv_indptr``/``kv_indices``: SGLang's int32 token (or
    page) index lists. ``num_kv_splits``: int32 ``[B]`` requested splits.
    ``attn_logits``/``attn_lse``: FP32 scratch ``[>=B, H, max_kv_splits + 1, D]``
    / ``[>=B, H, max_kv_splits + 1]``; every split slot a request uses is
    written (empty splits neutral), so no clearing launch is needed.
    ``req_pool_indices`` (int64 ``[B]``) locates the window ring rows; without a
    window (``has_hp=False``) it may be omitted.
    """
    li = layer_id - pool.start_layer
    B = q.shape[0]
    P, W = (pool._win_p, pool._win_r) if has_hp else (0, 0)
    if req_pool_indices is None:
        if P + W:
            raise ValueError("req_pool_indices is required when the BF16 window is enabled")
        req_pool_indices = torch.zeros(B, dtype=torch.int64, device=q.device)
    req = req_pool_indices.reshape(-1)
    if req.dtype != torch.int64:
        req = req.to(torch.int64)
    sl = None
    if seq_lens is not None:
        sl = seq_lens.reshape(-1)
        if sl.dtype != torch.int64:
            sl = sl.to(torch.int64)
    return kernels.decode_fwd(q, pool.c_codes[li], pool.c_params[li], pool.rope_buf[li], pool.hp_c[li],
                              kv_indptr, kv_indices, sl, req, num_kv_splits, max_kv_splits,
                              attn_logits, attn_lse, o, sm_scale, P, W, page_size,
                              max_reqs=pool._max_reqs if P + W else 0)
