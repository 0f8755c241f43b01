"""Drop-in extend (chunked prefill) reader over the packed pool (HIP implementation).

The patched SGLang hands the MLA attention, for an extend batch, the absorbed
query ``q = [q_nope_out | q_pe]`` in the rotated frame, the chunk's own keys
``k = [k_nope | k_pe]`` and the packed pool (deployment/patches/rolaq_sglang.patch:208-235);
the reader attends causally over the packed prefix and the chunk. The fork's
kernel is not in the reference; its row semantics are the HF cache's
(mla_quant/cache.py:1030-1039): INT2 rows dequantized to bf16, the first ``P``
and last ``W`` positions of the extended sequence as BF16 window rows, the
chunk's rows as given.
"""

from __future__ import annotations

import torch

from . import kernels


def packed_mla_extend_fwd(q, k, o, pool, layer_id, qo_indptr, kv_indptr, kv_indices, prefix_lens,
                          req_pool_indices, max_q_len, sm_scale, page_size: int = 1, workspace=None,
                          prefix_lens_cpu=None):
    """Extend attention of layer ``layer_id`` of ``pool``.

    ``q``: bf16 ``[T, H, D + R]``; ``k``: the chunk's keys, bf16 ``[T, D + R]``
    (or ``[T, 1, D + R]``); ``o``: bf16 ``[T, H, D]``. ``qo_indptr``: int32
    ``[B + 1]`` chunk offsets; ``kv_indptr``/``kv_indices``: the prefix's
    token (or page) lists; ``prefix_lens``/``req_pool_indices``: int64 ``[B]``.
    ``prefix_lens_cpu``: the prefix lengths on the host (SGLang's
    ``extend_prefix_lens_cpu``); with them the call needs no host sync, else
    it reads ``prefix_lens`` back once. ``workspace``: 16-bit ``[rows, D + R]``
    scratch with ``rows >= sum(prefix_lens) + T``; when omitted the pool's
    own workspace is used (kept across layers and calls, grown as needed).
    """
    li = layer_id - pool.start_layer
    if k.dim() == 3:
        k = k.reshape(k.shape[0], k.shape[-1])
    pl = prefix_lens.reshape(-1)
    if pl.dtype != torch.int64:
        pl = pl.to(torch.int64)
    req = req_pool_indices.reshape(-1)
    if req.dtype != torch.int64:
        req = req.to(torch.int64)
    B = qo_indptr.numel() - 1
    if prefix_lens_cpu is not None:
        key_rows = int(sum(int(v) for v in list(prefix_lens_cpu)[:B])) + int(q.shape[0])
    else:
        key_rows = int(pl[:B].sum().item()) + int(q.shape[0])
    if workspace is None:
        workspace = pool.extend_workspace(key_rows)
    return kernels.extend_fwd(q, k, qo_indptr, kv_indptr, kv_indices, pl, req, pool.c_codes[li], pool.c_params[li],
                              pool.rope_buf[li], pool.hp_c[li], max_q_len, o, sm_scale, pool._win_p, pool._win_r,
                              page_size, max_reqs=pool._max_reqs, workspace=workspace, key_rows=key_rows)
