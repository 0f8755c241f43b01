"""Tensor-level calls into the C ABI (``include/rolaq_mla.h``).

Each function checks devices, dtypes and layouts on the host, then passes raw
pointers and the current HIP stream of the tensors' device. No allocation,
no synchronisation, no host branch on device data.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

GROUP_SIZE = 128


def _p(t: torch.Tensor | None):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, device: torch.device, ndim: int | None = None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.device != device:
        raise ValueError(f"{name} must be on {device}, got {t.device}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims, got {tuple(t.shape)}")


def _contig(t: torch.Tensor, name: str):
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def scatter_pack_rows(x: torch.Tensor, slots: torch.Tensor, codes: torch.Tensor, params: torch.Tensor,
                      threshold: float, gain: float) -> None:
    """Quantize FP32 rotated rows ``x [n, D]`` into ``codes``/``params`` at ``slots``."""
    dev = x.device
    _need(x, "x", torch.float32, dev, 2)
    n, D = x.shape
    _need(slots, "slots", torch.int32, dev, 1)
    _need(codes, "codes", torch.uint8, dev, 2)
    _need(params, "params", torch.float32, dev, 3)
    if slots.numel() != n or codes.shape[1] != D // 4 or tuple(params.shape[1:]) != (D // GROUP_SIZE, 2):
        raise ValueError("scatter_pack_rows: shape mismatch")
    if x.stride(1) != 1:
        raise ValueError("x rows must be contiguous")
    _contig(slots, "slots"), _contig(codes, "codes"), _contig(params, "params")
    _lib.check(_lib.load().rolaq_scatter_pack_rows(
        _p(x), x.stride(0), _p(slots), n, D, GROUP_SIZE, float(threshold), float(gain),
        _p(codes), _p(params), _stream(x)))


def _check_writer(latent, k_pe, rotation_t, loc, seq_lens, positions, req_idx, codes, params, rope_buf, hp_c,
                  row_of_slot, owner_of_row, P, W, max_reqs) -> None:
    """Shape, dtype and device checks shared by the writer entry points."""
    dev = latent.device
    _need(latent, "latent", torch.bfloat16, dev, 2)
    n, D = latent.shape
    _need(k_pe, "k_pe", torch.bfloat16, dev, 2)
    R = k_pe.shape[1]
    if k_pe.shape[0] != n:
        raise ValueError("k_pe rows must match latent rows")
    if rotation_t is not None:
        _need(rotation_t, "rotation_t", torch.bfloat16, dev, 2)
        _contig(rotation_t, "rotation_t")
        if tuple(rotation_t.shape) != (D, D):
            raise ValueError("rotation_t must be [D, D]")
    for name, t in (("loc", loc), ("seq_lens", seq_lens), ("req_idx", req_idx)):
        _need(t, name, torch.int64, dev, 1)
        _contig(t, name)
        if t.numel() != n:
            raise ValueError(f"{name} must have {n} entries")
    if positions is not None:
        _need(positions, "positions", torch.int64, dev, 1)
        _contig(positions, "positions")
        if positions.numel() != n:
            raise ValueError("positions must have n entries")
    _need(codes, "codes", torch.uint8, dev, 2)
    _need(params, "params", torch.float32, dev, 3)
    _need(rope_buf, "rope_buf", torch.bfloat16, dev, 2)
    _need(hp_c, "hp_c", torch.bfloat16, dev, 2)
    _need(row_of_slot, "row_of_slot", torch.int32, dev, 1)
    _need(owner_of_row, "owner_of_row", torch.int32, dev, 1)
    for name, t in (("codes", codes), ("params", params), ("rope_buf", rope_buf), ("hp_c", hp_c),
                    ("row_of_slot", row_of_slot), ("owner_of_row", owner_of_row)):
        _contig(t, name)
    if codes.shape[1] != D // 4 or tuple(params.shape[1:]) != (D // GROUP_SIZE, 2) or rope_buf.shape[1] != R \
            or hp_c.shape[1] != D:
        raise ValueError("cache buffers do not match (D, R)")
    if hp_c.shape[0] < 1 + max_reqs * (P + W) or owner_of_row.shape[0] < 1 + max_reqs * (P + W):
        raise ValueError("hp_c / owner_of_row are smaller than 1 + max_reqs * (P + W)")
    if latent.stride(1) != 1:
        raise ValueError("latent rows must be contiguous")


def write_rows(latent: torch.Tensor, k_pe: torch.Tensor, rotation_t: torch.Tensor | None,
               loc: torch.Tensor, seq_lens: torch.Tensor, positions: torch.Tensor | None,
               req_idx: torch.Tensor, codes: torch.Tensor, params: torch.Tensor,
               rope_buf: torch.Tensor, hp_c: torch.Tensor, row_of_slot: torch.Tensor,
               owner_of_row: torch.Tensor, P: int, W: int, max_reqs: int,
               threshold: float, gain: float) -> None:
    """Fused rotate + quantize + pack + rope/window stores for ``n`` rows."""
    _check_writer(latent, k_pe, rotation_t, loc, seq_lens, positions, req_idx, codes, params, rope_buf, hp_c,
                  row_of_slot, owner_of_row, P, W, max_reqs)
    n, D = latent.shape
    R = k_pe.shape[1]
    _lib.check(_lib.load().rolaq_write_rows(
        _p(latent), latent.stride(0), _p(k_pe), k_pe.stride(0), k_pe.stride(1), _p(rotation_t),
        _p(loc), _p(seq_lens), _p(positions), _p(req_idx), n, D, R, int(P), int(W), int(max_reqs),
        float(threshold), float(gain), _p(codes), _p(params), _p(rope_buf), _p(hp_c),
        _p(row_of_slot), _p(owner_of_row), _stream(latent)))


def norm_write_rows(kv_a: torch.Tensor, norm_weight: torch.Tensor, eps: float, latent_out: torch.Tensor | None,
                    k_pe: torch.Tensor, rotation_t: torch.Tensor, loc: torch.Tensor, seq_lens: torch.Tensor,
                    positions: torch.Tensor | None, req_idx: torch.Tensor, codes: torch.Tensor, params: torch.Tensor,
                    rope_buf: torch.Tensor, hp_c: torch.Tensor, row_of_slot: torch.Tensor,
                    owner_of_row: torch.Tensor, P: int, W: int, max_reqs: int,
                    threshold: float, gain: float) -> None:
    """kv_a_layernorm + rotate + quantize + pack + rope/window stores for ``n`` rows.

    ``kv_a`` holds the pre-norm rows; ``latent_out`` (or None) receives the
    normalized bf16 rows. The cache arguments are those of :func:`write_rows`.
    """
    dev = kv_a.device
    _need(kv_a, "kv_a", torch.bfloat16, dev, 2)
    n, D = kv_a.shape
    _need(norm_weight, "norm_weight", torch.bfloat16, dev, 1)
    _contig(norm_weight, "norm_weight")
    if norm_weight.numel() != D:
        raise ValueError("norm_weight must have D entries")
    if rotation_t is None:
        raise ValueError("rotation_t is required (the identity for an un-rotated layer)")
    if latent_out is not None:
        _need(latent_out, "latent_out", torch.bfloat16, dev, 2)
        if tuple(latent_out.shape) != (n, D) or latent_out.stride(1) != 1:
            raise ValueError("latent_out must be [n, D] with contiguous rows")
    if not math.isfinite(eps) or eps < 0:
        raise ValueError("eps must be finite and >= 0")
    # the shared checks of write_rows, then the fused launch
    _check_writer(kv_a, k_pe, rotation_t, loc, seq_lens, positions, req_idx, codes, params, rope_buf, hp_c,
                  row_of_slot, owner_of_row, P, W, max_reqs)
    _lib.check(_lib.load().rolaq_norm_write_rows(
        _p(kv_a), kv_a.stride(0), _p(norm_weight), float(eps), _p(latent_out),
        latent_out.stride(0) if latent_out is not None else 0, _p(k_pe), k_pe.stride(0), k_pe.stride(1),
        _p(rotation_t), _p(loc), _p(seq_lens), _p(positions), _p(req_idx), n, D, k_pe.shape[1], int(P), int(W),
        int(max_reqs), float(threshold), float(gain), _p(codes), _p(params), _p(rope_buf), _p(hp_c),
        _p(row_of_slot), _p(owner_of_row), _stream(kv_a)))


def prepare_gf_splits(splits: torch.Tensor, quant: torch.Tensor, merge: torch.Tensor) -> None:
    """``quant = max(splits - 1, 1)``, ``merge = quant + 1`` in one launch."""
    dev = splits.device
    for name, t in (("splits", splits), ("quant", quant), ("merge", merge)):
        _need(t, name, torch.int32, dev)
        _contig(t, name)
        if t.numel() != splits.numel():
            raise ValueError("splits/quant/merge must have the same size")
    _lib.check(_lib.load().rolaq_prepare_gf_splits(_p(splits), _p(quant), _p(merge), splits.numel(),
                                                   _stream(splits)))


def _decode_check(q, codes, params, rope_buf, hp_c, kv_indptr, kv_indices, seq_lens, req_idx, num_kv_splits,
                  max_kv_splits, attn_logits, attn_lse):
    dev = q.device
    _need(q, "q", torch.bfloat16, dev, 3)
    B, H, DR = q.shape
    D = codes.shape[1] * 4
    R = DR - D
    if q.stride(2) != 1:
        raise ValueError("q must be contiguous in its last dim")
    _need(codes, "codes", torch.uint8, dev, 2)
    _need(params, "params", torch.float32, dev, 3)
    _need(rope_buf, "rope_buf", torch.bfloat16, dev, 2)
    _need(hp_c, "hp_c", torch.bfloat16, dev, 2)
    for name, t in (("codes", codes), ("params", params), ("rope_buf", rope_buf), ("hp_c", hp_c)):
        _contig(t, name)
    if rope_buf.shape[1] != R or hp_c.shape[1] != D or tuple(params.shape[1:]) != (D // GROUP_SIZE, 2):
        raise ValueError("cache buffers do not match q's (D, R)")
    _need(kv_indptr, "kv_indptr", torch.int32, dev, 1)
    _need(kv_indices, "kv_indices", torch.int32, dev, 1)
    _need(req_idx, "req_idx", torch.int64, dev, 1)
    _need(num_kv_splits, "num_kv_splits", torch.int32, dev, 1)
    for name, t in (("kv_indptr", kv_indptr), ("kv_indices", kv_indices), ("req_idx", req_idx),
                    ("num_kv_splits", num_kv_splits)):
        _contig(t, name)
    if kv_indptr.numel() < B + 1 or req_idx.numel() < B or num_kv_splits.numel() < B:
        raise ValueError("index tensors are shorter than the batch")
    if seq_lens is not None:
        _need(seq_lens, "seq_lens", torch.int64, dev, 1)
        _contig(seq_lens, "seq_lens")
        if seq_lens.numel() < B:
            raise ValueError("seq_lens is shorter than the batch")
    _scratch_check(attn_logits, attn_lse, B, H, D, max_kv_splits, dev)
    return B, H, D, R


def _ring_reqs(hp_c: torch.Tensor, P: int, W: int, max_reqs: int | None) -> int:
    """Requests whose ring rows ``hp_c`` holds (all of them when not given)."""
    width = int(P) + int(W)
    rows = hp_c.shape[0]
    if max_reqs is None:
        return (rows - 1) // width if width else 0
    max_reqs = int(max_reqs)
    if max_reqs < 0:
        raise ValueError("max_reqs must be >= 0")
    if width and rows < 1 + max_reqs * width:
        raise ValueError(f"hp_c has {rows} rows, fewer than 1 + max_reqs * (P + W) = {1 + max_reqs * width}")
    return max_reqs


def _scratch_check(attn_logits, attn_lse, B, H, D, max_kv_splits, dev):
    S1 = int(max_kv_splits) + 1
    _need(attn_logits, "attn_logits", torch.float32, dev)
    _need(attn_lse, "attn_lse", torch.float32, dev)
    _contig(attn_logits, "attn_logits"), _contig(attn_lse, "attn_lse")
    if tuple(attn_logits.shape[1:]) != (H, S1, D) or attn_logits.shape[0] < B \
            or tuple(attn_lse.shape[1:]) != (H, S1) or attn_lse.shape[0] < B:
        raise ValueError("attn_logits / attn_lse must be [>=B, H, max_kv_splits + 1, (D)]")


def _out_check(out, B, H, D, dev):
    _need(out, "out", torch.bfloat16, dev, 3)
    if tuple(out.shape) != (B, H, D) or out.stride(2) != 1:
        raise ValueError("out must be [B, H, D] with a contiguous last dim")


def decode_fwd(q: torch.Tensor, codes: torch.Tensor, params: torch.Tensor, rope_buf: torch.Tensor,
               hp_c: torch.Tensor, kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
               seq_lens: torch.Tensor | None, req_idx: torch.Tensor, num_kv_splits: torch.Tensor,
               max_kv_splits: int, attn_logits: torch.Tensor, attn_lse: torch.Tensor,
               out: torch.Tensor, sm_scale: float, P: int, W: int, page_size: int = 1,
               max_reqs: int | None = None) -> torch.Tensor:
    """Absorbed decode over the packed cache: ``q [B, H, D+R]`` -> ``out [B, H, D]``.

    ``max_reqs``: requests with ring rows in ``hp_c`` (default: as many as its
    rows hold); a ``req_idx`` outside ``[0, max_reqs)`` reads no window rows.
    Request ``b`` uses ``min(num_kv_splits[b], decode_split_cap(...))`` splits
    (about one working block per compute unit); the partials in
    ``attn_logits``/``attn_lse`` follow that count."""
    B, H, D, R = _decode_check(q, codes, params, rope_buf, hp_c, kv_indptr, kv_indices, seq_lens, req_idx,
                               num_kv_splits, max_kv_splits, attn_logits, attn_lse)
    _out_check(out, B, H, D, q.device)
    mr = _ring_reqs(hp_c, P, W, max_reqs)
    _lib.check(_lib.load().rolaq_decode_fwd(
        _p(q), q.stride(0), q.stride(1), _p(codes), _p(params), _p(rope_buf), _p(hp_c),
        _p(kv_indptr), _p(kv_indices), int(page_size), _p(seq_lens), _p(req_idx), mr, _p(num_kv_splits),
        int(max_kv_splits), B, H, D, R, int(P), int(W), float(sm_scale), _p(attn_logits),
        _p(attn_lse), _p(out), out.stride(0), out.stride(1), _stream(q)))
    return out


def decode_split_cap(B: int, H: int, D: int, max_kv_splits: int) -> int:
    """The most splits :func:`decode_fwd` gives one request on the current
    device: enough quantized splits for one working block per compute unit
    over the batch, plus the window split, at most ``max_kv_splits``."""
    cap = ctypes.c_int(0)
    _lib.check(_lib.load().rolaq_decode_split_cap(int(B), int(H), int(D), int(max_kv_splits), ctypes.byref(cap)))
    return cap.value


def decode_partials(q: torch.Tensor, codes: torch.Tensor, params: torch.Tensor, rope_buf: torch.Tensor,
                    hp_c: torch.Tensor, kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                    seq_lens: torch.Tensor | None, req_idx: torch.Tensor, num_kv_splits: torch.Tensor,
                    max_kv_splits: int, attn_logits: torch.Tensor, attn_lse: torch.Tensor,
                    sm_scale: float, P: int, W: int, page_size: int = 1, max_reqs: int | None = None) -> None:
    """Stage 1 of :func:`decode_fwd` alone: fills ``attn_logits`` / ``attn_lse``."""
    B, H, D, R = _decode_check(q, codes, params, rope_buf, hp_c, kv_indptr, kv_indices, seq_lens, req_idx,
                               num_kv_splits, max_kv_splits, attn_logits, attn_lse)
    mr = _ring_reqs(hp_c, P, W, max_reqs)
    _lib.check(_lib.load().rolaq_decode_partials(
        _p(q), q.stride(0), q.stride(1), _p(codes), _p(params), _p(rope_buf), _p(hp_c),
        _p(kv_indptr), _p(kv_indices), int(page_size), _p(seq_lens), _p(req_idx), mr, _p(num_kv_splits),
        int(max_kv_splits), B, H, D, R, int(P), int(W), float(sm_scale), _p(attn_logits),
        _p(attn_lse), _stream(q)))


def decode_merge(attn_logits: torch.Tensor, attn_lse: torch.Tensor, num_kv_splits: torch.Tensor,
                 max_kv_splits: int, out: torch.Tensor) -> torch.Tensor:
    """Stage 2 of :func:`decode_fwd` alone: LSE merge of the partials into ``out [B, H, D]``."""
    dev = out.device
    _need(num_kv_splits, "num_kv_splits", torch.int32, dev, 1)
    _contig(num_kv_splits, "num_kv_splits")
    B, H, D = out.shape
    if num_kv_splits.numel() < B:
        raise ValueError("num_kv_splits is shorter than the batch")
    _scratch_check(attn_logits, attn_lse, B, H, D, max_kv_splits, dev)
    _out_check(out, B, H, D, dev)
    _lib.check(_lib.load().rolaq_decode_merge(
        _p(attn_logits), _p(attn_lse), _p(num_kv_splits), int(max_kv_splits), B, H, D, _p(out),
        out.stride(0), out.stride(1), _stream(out)))
    return out


def extend_fwd(q: torch.Tensor, k_chunk: torch.Tensor, qo_indptr: torch.Tensor, kv_indptr: torch.Tensor,
               kv_indices: torch.Tensor, prefix_lens: torch.Tensor, req_idx: torch.Tensor, codes: torch.Tensor,
               params: torch.Tensor, rope_buf: torch.Tensor, hp_c: torch.Tensor, max_q_len: int,
               out: torch.Tensor, sm_scale: float, P: int, W: int, page_size: int = 1,
               max_reqs: int | None = None, workspace: torch.Tensor | None = None,
               key_rows: int | None = None) -> torch.Tensor:
    """Causal extend over the packed prefix + the chunk: ``q [T, H, D+R]`` -> ``out [T, H, D]``.

    ``max_reqs`` as for :func:`decode_fwd`. ``key_rows``: the number of key
    rows of the extended sequences, ``sum(prefix_lens) + T``, as the caller
    knows it on the host (SGLang: ``extend_prefix_lens_cpu`` and the token
    count); read back from the device when not given (one host sync).
    ``workspace``: 16-bit ``[rows, D + R]`` scratch (bf16 or fp16 storage;
    fp16 values are written into it) with ``rows >= key_rows``, allocated
    here when not given; a shorter one raises ``ValueError``."""
    dev = q.device
    _need(q, "q", torch.bfloat16, dev, 3)
    T, H, DR = q.shape
    D = codes.shape[1] * 4
    R = DR - D
    if q.stride(2) != 1:
        raise ValueError("q must be contiguous in its last dim")
    _need(k_chunk, "k_chunk", torch.bfloat16, dev, 2)
    if k_chunk.shape[0] < T or k_chunk.shape[1] != DR or k_chunk.stride(1) != 1:
        raise ValueError("k_chunk must be [T, D + R] with a contiguous last dim")
    _need(codes, "codes", torch.uint8, dev, 2)
    _need(params, "params", torch.float32, dev, 3)
    _need(rope_buf, "rope_buf", torch.bfloat16, dev, 2)
    _need(hp_c, "hp_c", torch.bfloat16, dev, 2)
    for name, t in (("codes", codes), ("params", params), ("rope_buf", rope_buf), ("hp_c", hp_c)):
        _contig(t, name)
    if rope_buf.shape[1] != R or hp_c.shape[1] != D or tuple(params.shape[1:]) != (D // GROUP_SIZE, 2):
        raise ValueError("cache buffers do not match q's (D, R)")
    for name, t, dt in (("qo_indptr", qo_indptr, torch.int32), ("kv_indptr", kv_indptr, torch.int32),
                        ("kv_indices", kv_indices, torch.int32), ("prefix_lens", prefix_lens, torch.int64),
                        ("req_idx", req_idx, torch.int64)):
        _need(t, name, dt, dev, 1)
        _contig(t, name)
    B = qo_indptr.numel() - 1
    if B < 0 or kv_indptr.numel() < B + 1 or prefix_lens.numel() < B or req_idx.numel() < B:
        raise ValueError("index tensors are shorter than the batch")
    _need(out, "out", torch.bfloat16, dev, 3)
    if out.shape[0] < T or tuple(out.shape[1:]) != (H, D) or out.stride(2) != 1:
        raise ValueError("out must be [T, H, D] with a contiguous last dim")
    mr = _ring_reqs(hp_c, P, W, max_reqs)
    if key_rows is None:
        key_rows = int(prefix_lens[:B].sum().item()) + int(qo_indptr[B].item()) - int(qo_indptr[0].item())
    if workspace is None:
        workspace = torch.empty(max(int(key_rows), 1), DR, dtype=torch.float16, device=dev)
    if workspace.dtype not in (torch.bfloat16, torch.float16) or workspace.device != dev or workspace.dim() != 2:
        raise TypeError("workspace must be a 2-D bf16 or fp16 tensor on the query's device")
    _contig(workspace, "workspace")
    if workspace.shape[1] != DR:
        raise ValueError("workspace must be [rows, D + R]")
    _lib.check(_lib.load().rolaq_extend_fwd(
        _p(q), q.stride(0), q.stride(1), _p(k_chunk), k_chunk.stride(0), _p(qo_indptr), _p(kv_indptr),
        _p(kv_indices), int(page_size), _p(prefix_lens), _p(req_idx), mr, _p(codes), _p(params), _p(rope_buf),
        _p(hp_c), B, H, D, R, int(P), int(W), int(max_q_len), float(sm_scale), _p(workspace),
        workspace.shape[0], int(key_rows), _p(out), out.stride(0), out.stride(1), _stream(q)))
    return out


def assemble_rows(slots: torch.Tensor, codes: torch.Tensor, params: torch.Tensor, rope_buf: torch.Tensor,
                  hp_c: torch.Tensor, row_of_slot: torch.Tensor, owner_of_row: torch.Tensor,
                  rotation: torch.Tensor | None, out: torch.Tensor) -> torch.Tensor:
    """Cache rows at ``slots`` as bf16 ``[n, D + R]`` (latent, optionally un-rotated, then rope)."""
    dev = codes.device
    _need(slots, "slots", torch.int64, dev, 1)
    _contig(slots, "slots")
    D = codes.shape[1] * 4
    R = rope_buf.shape[1]
    for name, t, dt in (("codes", codes, torch.uint8), ("params", params, torch.float32),
                        ("rope_buf", rope_buf, torch.bfloat16), ("hp_c", hp_c, torch.bfloat16),
                        ("row_of_slot", row_of_slot, torch.int32), ("owner_of_row", owner_of_row, torch.int32)):
        _need(t, name, dt, dev)
        _contig(t, name)
    if hp_c.shape[1] != D or tuple(params.shape[1:]) != (D // GROUP_SIZE, 2):
        raise ValueError("cache buffers do not match")
    if rotation is not None:
        _need(rotation, "rotation", torch.bfloat16, dev, 2)
        _contig(rotation, "rotation")
        if tuple(rotation.shape) != (D, D):
            raise ValueError("rotation must be [D, D]")
    _need(out, "out", torch.bfloat16, dev, 2)
    if out.shape[0] < slots.numel() or out.shape[1] < D + R or out.stride(1) != 1:
        raise ValueError("out must be [n, >= D + R] with a contiguous last dim")
    _lib.check(_lib.load().rolaq_assemble_rows(
        _p(slots), slots.numel(), _p(codes), _p(params), _p(rope_buf), _p(hp_c), _p(row_of_slot),
        _p(owner_of_row), _p(rotation), D, R, _p(out), out.stride(0), _stream(codes)))
    return out
