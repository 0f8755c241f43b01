"""Cache rows of the packed pool as bf16 ``[latent | rope]`` rows (HIP implementation).

For MHA-style prefill over a packed prefix: the fork's ``_assemble_rows_kernel``
(deployment/patches/rolaq_sglang.patch:5-6) writes ``[latent | rope]`` per row,
and ``kv_b_proj`` consumes the latent in the model's (un-rotated) frame
(deployment/sglang/srt/mem_cache/rolaq_mla.py:60-61).
"""

from __future__ import annotations

import torch

from . import kernels


def assemble_rows(pool, layer_id, slots, out=None, unrotate: bool = True):
    """Rows at ``slots`` of layer ``layer_id``: bf16 ``[n, D + R]``.

    The latent is the window row while the slot owns one, else the dequantized
    INT2 row; with ``unrotate`` (and a rotation on the layer) it is multiplied
    back by ``R_eff^T`` -- ``rotate_quantize``'s restored value for INT2 rows.
    """
    li = layer_id - pool.start_layer
    D, R = pool.kv_lora_rank, pool.qk_rope_head_dim
    s = slots.reshape(-1)
    if s.dtype != torch.int64:
        s = s.to(torch.int64)
    s = s.contiguous()
    if out is None:
        out = torch.empty(s.numel(), D + R, dtype=torch.bfloat16, device=pool.c_codes[li].device)
    rot = pool.latent_rotation(layer_id, local=True) if unrotate else None
    if rot is not None and rot.dtype != torch.bfloat16:
        rot = rot.to(torch.bfloat16)
    return kernels.assemble_rows(s, pool.c_codes[li], pool.c_params[li], pool.rope_buf[li], pool.hp_c[li],
                                 pool.hp_row_of_slot, pool.hp_owner_of_row,
                                 None if rot is None else rot.contiguous(), out)
