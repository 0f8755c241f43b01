"""Drop-in writer entry points (reference interface, HIP implementation).

``try_fast_decode_store`` mirrors deployment/sglang/QuantKernel/mla_fused_writer.py:110-224
(same gatekeeping, same pool attributes read and written, ``False`` means "not
handled"); ``scatter_pack_rows`` mirrors deployment/patches/rolaq_sglang.patch:9-34.
Both call the fused HIP kernels of ``librolaq_mla.so``.
"""

from __future__ import annotations

import torch

from . import kernels

# OSCAR defaults (mla_quant/oscar.py:104,111) used when a layer has no learned (t, g).
LM_THRESHOLD = 0.9810652732849121
LM_GAIN = 1.16
SUPPORTED_DIMS = {(512, 64), (256, 32)}


def _as_int64(t: torch.Tensor) -> torch.Tensor:
    t = t.reshape(-1)
    return t if t.dtype == torch.int64 and t.is_contiguous() else t.to(torch.int64).contiguous()


def _write_rotation(pool, layer_id: int, r: torch.Tensor | None):
    """bf16 R_eff^T for the kernel, cached per layer and keyed by the identity of
    the pool's rotation object (mla_fused_writer.py:137-149 asserts it never changes)."""
    cached = getattr(pool, "_fast_write_rotation", None)
    if cached is None:
        cached = pool._fast_write_rotation = {}
    if r is None:
        return None
    if layer_id not in cached:
        cached[layer_id] = (id(r), r.to(torch.bfloat16).t().contiguous())
    assert cached[layer_id][0] == id(r)
    return cached[layer_id][1]


def _identity_rotation(pool, device) -> torch.Tensor:
    """bf16 identity for un-rotated layers on the fused-norm path (x * I is exact)."""
    eye = getattr(pool, "_fast_write_identity", None)
    if eye is None:
        eye = pool._fast_write_identity = torch.eye(pool.kv_lora_rank, dtype=torch.bfloat16, device=device)
    return eye


def _decode_handled(pool, n: int) -> bool:
    """The gatekeeping of mla_fused_writer.py:117-134 for a decode step of ``n`` rows."""
    meta = pool._fb_window_meta
    if (
        n <= 0
        or (pool.kv_lora_rank, pool.qk_rope_head_dim) not in SUPPORTED_DIMS
        or not pool._latent_windows
        or not meta
        or meta.get("fallback")
        or not meta["is_decode"]
        or meta["seq_lens"] is None
        or meta["req_pool_indices"] is None
        or meta["seq_lens"].numel() != n
        or meta["req_pool_indices"].numel() != n
        or pool._selfcheck_budget > 0
        or pool._audit_budget > 0
    ):
        return False
    return bool(pool._lloyd_max and pool._bits == 2)


def try_fast_decode_store(pool, layer_id, loc, c_kv, k_pe) -> bool:
    """Return whether the decode write was handled; the caller falls back otherwise.

    One launch rotates (bf16 MFMA), quantizes, packs and stores rope, window row
    and ring ownership for every row of this decode step.
    """
    meta = pool._fb_window_meta
    if not _decode_handled(pool, c_kv.numel() // pool.kv_lora_rank):
        return False
    li = layer_id - pool.start_layer
    r = pool.latent_rotation(layer_id, local=True)
    rt = _write_rotation(pool, layer_id, r)
    frames = getattr(pool, "_rot_write_frame", None)
    if frames is None:
        frames = pool._rot_write_frame = {}
    if r is not None:
        frames.setdefault(layer_id, id(r))
    loc64 = _as_int64(loc)
    pool._write_loc = loc64
    x = c_kv.reshape(-1, pool.kv_lora_rank)
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    pe = k_pe.reshape(-1, pool.qk_rope_head_dim)
    params = pool._rolaq_quantizers[li]
    t, g = (params[0], params[1]) if params is not None else (LM_THRESHOLD, LM_GAIN)
    kernels.write_rows(
        x, pe, rt, loc64, _as_int64(meta["seq_lens"]), None, _as_int64(meta["req_pool_indices"]),
        pool.c_codes[li], pool.c_params[li], pool.rope_buf[li], pool.hp_c[li], pool.hp_row_of_slot,
        pool.hp_owner_of_row, pool._win_p, pool._win_r, pool._max_reqs, t, g)
    return True


def write_prefill(pool, layer_id, loc, c_kv, k_pe, positions, seq_lens, req_pool_indices) -> None:
    """Prefill / chunked-prefill write of ``n`` rows with explicit positions.

    The reference runs rotate -> scatter_pack_rows -> ``rope_buf[loc] = pe`` and
    leaves the window stores to the fork's pool (rolaq_sglang.patch:155-164);
    here one launch does all of it with the decode writer's keep/ring rule,
    ``seq_lens`` being each row's sequence length after this chunk.
    """
    li = layer_id - pool.start_layer
    r = pool.latent_rotation(layer_id, local=True)
    rt = _write_rotation(pool, layer_id, r)
    x = c_kv.reshape(-1, pool.kv_lora_rank)
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    pe = k_pe.reshape(-1, pool.qk_rope_head_dim)
    params = pool._rolaq_quantizers[li]
    t, g = (params[0], params[1]) if params is not None else (LM_THRESHOLD, LM_GAIN)
    kernels.write_rows(
        x, pe, rt, _as_int64(loc), _as_int64(seq_lens), _as_int64(positions), _as_int64(req_pool_indices),
        pool.c_codes[li], pool.c_params[li], pool.rope_buf[li], pool.hp_c[li], pool.hp_row_of_slot,
        pool.hp_owner_of_row, pool._win_p, pool._win_r, pool._max_reqs, t, g)


def _quantizer(pool, li: int):
    params = pool._rolaq_quantizers[li]
    return (params[0], params[1]) if params is not None else (LM_THRESHOLD, LM_GAIN)


def try_fast_norm_decode_store(pool, layer_id, loc, kv_a, k_pe, norm_weight, eps, latent_out=None) -> bool:
    """``try_fast_decode_store(pool, layer_id, loc, kv_a_layernorm(kv_a), k_pe)`` in one launch.

    ``kv_a`` is the pre-norm compressed latent; ``norm_weight``/``eps`` are the
    layer's ``kv_a_layernorm`` (DeepseekV2RMSNorm) weight (bf16 [D]) and
    epsilon. ``latent_out`` ([n, D] bf16, or None) receives the normalized rows.
    Same gatekeeping as :func:`try_fast_decode_store`; ``False`` = not handled.
    """
    meta = pool._fb_window_meta
    if not _decode_handled(pool, kv_a.numel() // pool.kv_lora_rank):
        return False
    li = layer_id - pool.start_layer
    r = pool.latent_rotation(layer_id, local=True)
    rt = _write_rotation(pool, layer_id, r)
    if rt is None:
        rt = _identity_rotation(pool, kv_a.device)
    loc64 = _as_int64(loc)
    pool._write_loc = loc64
    x = kv_a.reshape(-1, pool.kv_lora_rank)
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    t, g = _quantizer(pool, li)
    kernels.norm_write_rows(
        x, norm_weight, float(eps), latent_out, k_pe.reshape(-1, pool.qk_rope_head_dim), rt, loc64,
        _as_int64(meta["seq_lens"]), None, _as_int64(meta["req_pool_indices"]), pool.c_codes[li],
        pool.c_params[li], pool.rope_buf[li], pool.hp_c[li], pool.hp_row_of_slot, pool.hp_owner_of_row,
        pool._win_p, pool._win_r, pool._max_reqs, t, g)
    return True


def norm_write_prefill(pool, layer_id, loc, kv_a, k_pe, positions, seq_lens, req_pool_indices, norm_weight, eps,
                       latent_out=None) -> None:
    """:func:`write_prefill` of ``kv_a_layernorm(kv_a)`` in one launch (see
    :func:`try_fast_norm_decode_store` for the norm arguments)."""
    li = layer_id - pool.start_layer
    r = pool.latent_rotation(layer_id, local=True)
    rt = _write_rotation(pool, layer_id, r)
    if rt is None:
        rt = _identity_rotation(pool, kv_a.device)
    x = kv_a.reshape(-1, pool.kv_lora_rank)
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    t, g = _quantizer(pool, li)
    kernels.norm_write_rows(
        x, norm_weight, float(eps), latent_out, k_pe.reshape(-1, pool.qk_rope_head_dim), rt, _as_int64(loc),
        _as_int64(seq_lens), _as_int64(positions), _as_int64(req_pool_indices), pool.c_codes[li],
        pool.c_params[li], pool.rope_buf[li], pool.hp_c[li], pool.hp_row_of_slot, pool.hp_owner_of_row,
        pool._win_p, pool._win_r, pool._max_reqs, t, g)


def scatter_pack_rows(x, slots, codes_buf, params_buf, group_size, lloyd_max, bits=2, quantizer_params=None):
    """Quantize ``x`` (``[n, D]``, rotated frame) into ``codes/params`` at ``slots``."""
    if not lloyd_max or bits != 2:
        if quantizer_params is not None:
            raise ValueError("Learned threshold/gain require the INT2 Lloyd writer")
        raise ValueError("this build implements the INT2 Lloyd codec only")
    if group_size != kernels.GROUP_SIZE:
        raise ValueError("group_size must be 128")
    n = x.shape[0]
    if n == 0:
        return
    x = x.contiguous().to(torch.float32)
    if quantizer_params is not None:
        threshold, gain = quantizer_params
    else:
        threshold, gain = LM_THRESHOLD, LM_GAIN
    slots32 = slots.reshape(-1)
    if slots32.dtype != torch.int32 or not slots32.is_contiguous():
        slots32 = slots32.to(torch.int32).contiguous()
    kernels.scatter_pack_rows(x, slots32, codes_buf, params_buf, threshold, gain)
