"""Oracle: absorbed MLA attention over the packed cache (dequantize, then attend).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Semantics follow the reference's HF fake-quant path, which is the only
complete in-tree statement of the arithmetic:
* cache rows are the rotated latent, FP32 Lloyd QDQ rounded to BF16
  (``mla_quant/quantizer.py:117-121``) except the first P / last W valid rows,
  which stay BF16 (``mla_quant/cache.py:775-800,1007-1073``);
* attention is eager BF16-input attention with an FP32 softmax
  (transformers ``modeling_deepseek_v2.py`` ``eager_attention_forward``,
  ``DeepseekV2Attention.forward``), written in the absorbed form the serving
  reader uses: ``s_t = scale * (q_lat . c_t + q_rope . kr_t)``, ``o = softmax(s) @ c``
  in the rotated latent frame (``deployment/patches/rolaq_sglang.patch:195-248``);
* split-K partials are merged with the log-sum-exp rule of SGLang's decode
  stage 2, empty splits carrying ``lse = -1e4`` and zero logits
  (``rolaq_sglang.patch:62-111``).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import codec, layout, window

NEUTRAL_LSE = -1.0e4


def bf16_bits_to_float(bits: np.ndarray) -> torch.Tensor:
    """Decode uint16 bf16 bit patterns into an FP32 tensor."""
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return torch.from_numpy(b.view(np.float32).copy())


def float_to_bf16_bits(x: torch.Tensor) -> np.ndarray:
    """Round to bf16 (nearest even) and return the uint16 bit patterns."""
    return x.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def gather_rows(pool: dict, slots, req: int, length: int, P: int, W: int,
                width: int, round_bf16: bool = True, max_reqs: int | None = None):
    """Cache rows of one sequence (positions ``0 .. length-1``) as FP32.

    Quantized positions are dequantized from ``codes/params`` (optionally
    rounded to bf16, as the reference's QDQ output is); window positions read
    ``hp`` at their ring row. A request outside ``[0, max_reqs)`` has no ring
    rows (the writer keeps none for it, ``mla_fused_writer.py:41``), so all
    its positions are dequantized. Returns ``(latent [L, D], rope [L, R])``.
    """
    if max_reqs is not None and not 0 <= int(req) < int(max_reqs):
        P = W = 0
    slots = np.asarray(slots, dtype=np.int64)[:length]
    pos = np.arange(length)
    codes = layout.unpack_codes(pool["codes"][slots], width)
    params = torch.from_numpy(pool["params"][slots])
    lat = codec.dequantize(torch.from_numpy(codes), params[..., 0], params[..., 1])
    if round_bf16:
        lat = lat.to(torch.bfloat16).float()
    hp_mask = window.positional_bf16(pos, length, P, W)
    if hp_mask.any():
        ring = window.ring_row(np.full(length, req), pos, P, W)[hp_mask]
        lat[torch.from_numpy(hp_mask)] = bf16_bits_to_float(pool["hp"][ring])
    rope = bf16_bits_to_float(pool["rope"][slots])
    return lat, rope


def attend(q_lat, q_rope, k_lat, k_rope, sm_scale: float, dtype=torch.float32, mask=None):
    """Absorbed attention for one sequence. ``q_*``: [T, H, *], ``k_*``: [L, *].

    Returns ``(out [T, H, D], lse [T, H])`` in ``dtype``; ``lse`` is natural-log.
    ``mask`` ([T, L] bool, True = visible) implements causality.
    """
    ql, qr = q_lat.to(dtype), q_rope.to(dtype)
    kl, kr = k_lat.to(dtype), k_rope.to(dtype)
    s = (torch.einsum("thd,ld->thl", ql, kl) + torch.einsum("thr,lr->thl", qr, kr)) * sm_scale
    if mask is not None:
        s = s.masked_fill(~mask[:, None, :], float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse[..., None])
    return torch.einsum("thl,ld->thd", p, kl), lse


def attend_bf16_eager(q_lat, q_rope, k_lat, k_rope, sm_scale: float, mask=None):
    """transformers eager path: bf16 matmuls (bf16 logits), FP32 softmax cast
    back to bf16, bf16 output (``eager_attention_forward``)."""
    q = torch.cat([q_lat, q_rope], -1).to(torch.bfloat16).transpose(0, 1)  # [H, T, D+R]
    k = torch.cat([k_lat, k_rope], -1).to(torch.bfloat16)  # [L, D+R]
    v = k_lat.to(torch.bfloat16)
    w = torch.matmul(q, k.T.contiguous()) * sm_scale
    if mask is not None:
        w = w.masked_fill(~mask[None], float("-inf"))
    p = torch.softmax(w, dim=-1, dtype=torch.float32).to(torch.bfloat16)
    return torch.matmul(p, v).transpose(0, 1)  # [T, H, D]


def decode(pool: dict, q_lat, q_rope, slots_per_seq, lengths, reqs, P: int, W: int,
           sm_scale: float, width: int, flavour: str = "fp32", max_reqs: int | None = None,
           batch_index=None):
    """Decode attention for a batch (one query token per sequence).

    ``flavour``: ``"stored64"`` (the reference's stored rows: INT2 rows
    dequantized in FP32 and rounded to bf16, window rows as stored; float64
    arithmetic), ``"fp32"`` (the same rows, FP32 logits/softmax), ``"fp64"``
    (exact FP32 dequant without the bf16 rounding, float64) or
    ``"bf16_eager"`` (transformers eager numerics). Returns ``[B, H, D]`` and
    the natural-log LSE ``[B, H]`` (nan for ``bf16_eager``), float64 for the
    float64 flavours. ``batch_index``: evaluate only these sequences (others
    stay zero).
    """
    B, H, _ = q_lat.shape
    wide = flavour in ("fp64", "stored64")
    out = torch.zeros(B, H, width, dtype=torch.float64 if wide else torch.float32)
    lses = torch.full((B, H), float("nan"), dtype=out.dtype)
    for b in (range(B) if batch_index is None else batch_index):
        L = int(lengths[b])
        if L == 0:
            continue
        k_lat, k_rope = gather_rows(pool, slots_per_seq[b], int(reqs[b]), L, P, W, width,
                                    round_bf16=(flavour != "fp64"), max_reqs=max_reqs)
        ql, qr = q_lat[b:b + 1].float(), q_rope[b:b + 1].float()
        if flavour == "bf16_eager":
            out[b] = attend_bf16_eager(ql, qr, k_lat, k_rope, sm_scale)[0].float()
        else:
            dt = torch.float64 if wide else torch.float32
            o, lse = attend(ql, qr, k_lat, k_rope, sm_scale, dt)
            out[b], lses[b] = o[0].to(out.dtype), lse[0].to(out.dtype)
    return out, lses


def merge_splits(parts: torch.Tensor, lses: torch.Tensor) -> torch.Tensor:
    """SGLang decode stage 2: ``o = sum_s e^{lse_s - m} o_s / sum_s e^{lse_s - m}``.

    ``parts``: [..., S, D] per-split normalised outputs, ``lses``: [..., S].
    """
    m = lses.max(dim=-1, keepdim=True).values
    w = torch.exp(lses - m)
    return (w[..., None] * parts).sum(-2) / w.sum(-1, keepdim=True)


def split_partials(q_lat, q_rope, k_lat, k_rope, sm_scale: float, bounds, dtype=torch.float64):
    """Per-split normalised outputs and LSEs for key ranges ``bounds`` (pairs);
    an empty range yields the neutral partial (zeros, ``NEUTRAL_LSE``)."""
    parts, lses = [], []
    H, D = q_lat.shape[-2], k_lat.shape[-1]
    for lo, hi in bounds:
        if hi <= lo:
            parts.append(torch.zeros(1, H, D, dtype=dtype))
            lses.append(torch.full((1, H), NEUTRAL_LSE, dtype=dtype))
            continue
        o, lse = attend(q_lat, q_rope, k_lat[lo:hi], k_rope[lo:hi], sm_scale, dtype)
        parts.append(o)
        lses.append(lse)
    return torch.stack(parts, -2), torch.stack(lses, -1)


def chunk_rows(chunk_lat, prefix_len: int, P: int, W: int, chunk_mode: str = "bf16",
               threshold: float = codec.LLOYD_MAX_THRESHOLD, gain: float = codec.LLOYD_MAX_STRETCH):
    """The chunk's key rows (FP32) as the extend attention sees them.

    ``"bf16"``: the given rows (SGLang extend semantics, rolaq_sglang.patch:208-235).
    ``"qdq"`` (HF semantics, mla_quant/cache.py:1028-1039: the chunk is written
    to the cache before attention): rows of the extended sequence's window
    (first ``P`` / last ``W`` positions) are its BF16 rows, the others the
    Lloyd QDQ of the row (``chunk_lat`` in FP32, the rotated latent) rounded to
    bf16, as the cache stores them (oscar.py:120-144, quantizer.py:117-120).
    """
    c_lat = chunk_lat.float()
    if chunk_mode == "qdq":
        L = prefix_len + c_lat.shape[0]
        pos = np.arange(prefix_len, L)
        quant = torch.from_numpy(~window.positional_bf16(pos, L, P, W))
        c_lat = c_lat.to(torch.bfloat16).float()
        if quant.any():
            _, _, _, qdq = codec.lloyd_codec(chunk_lat.float()[quant], codec.GROUP_SIZE, threshold, gain)
            c_lat[quant] = qdq.to(torch.bfloat16).float()
    return c_lat


def extend(pool: dict, q_lat, q_rope, chunk_lat, chunk_rope, prefix_slots, prefix_len: int,
           req: int, P: int, W: int, sm_scale: float, width: int, chunk_mode: str = "bf16",
           rotation=None, threshold: float = codec.LLOYD_MAX_THRESHOLD,
           gain: float = codec.LLOYD_MAX_STRETCH, dtype=torch.float32, max_reqs: int | None = None,
           rows=None, flavour: str = "fp"):
    """Causal extend attention of one sequence: ``Tq`` new queries at positions
    ``prefix_len ..`` over the packed prefix plus the chunk itself. A request
    outside ``[0, max_reqs)`` has no window rows (``P = W = 0``).

    ``chunk_mode="bf16"`` (SGLang extend semantics, rolaq_sglang.patch:208-235):
    the chunk's own rows enter as the given BF16 rotated latent.
    ``chunk_mode="qdq"`` (HF semantics, cache.py:1028-1039): chunk rows outside
    the window are Lloyd-QDQ'd (rounded to bf16) before attention, window rows
    rounded to bf16 (:func:`chunk_rows`).
    ``rows``: evaluate only the queries of these chunk rows (returns ``[len(rows), H, D]``).
    ``flavour="bf16_eager"``: the reference model's attention in bf16
    (:func:`attend_bf16_eager`; returns ``(out, None)``) instead of ``dtype``.
    """
    if max_reqs is not None and not 0 <= int(req) < int(max_reqs):
        P = W = 0
    Tq = q_lat.shape[0]
    L = prefix_len + Tq
    lat_p, rope_p = gather_rows(pool, prefix_slots, req, prefix_len, P, W, width)
    # Positional window with the *current* length: prefix rows inside the last
    # W positions (only when Tq < W) stay BF16; sinks stay BF16.
    if prefix_len:
        pos = np.arange(prefix_len)
        now_bf16 = window.positional_bf16(pos, L, P, W)
        was_bf16 = window.positional_bf16(pos, prefix_len, P, W)
        leave = torch.from_numpy(was_bf16 & ~now_bf16)
        if leave.any():
            # rows that left the window are read back from their INT2 codes
            lat_q, _ = gather_rows(pool, prefix_slots, req, prefix_len, 0, 0, width)
            lat_p[leave] = lat_q[leave]
    c_lat = chunk_rows(chunk_lat, prefix_len, P, W, chunk_mode, threshold, gain)
    k_lat = torch.cat([lat_p, c_lat], 0)
    k_rope = torch.cat([rope_p, chunk_rope.float()], 0)
    qpos = torch.arange(prefix_len, L)[:, None]
    kpos = torch.arange(L)[None, :]
    if rows is not None:  # only these chunk rows' queries (the keys are the whole chunk's)
        rows = torch.as_tensor(rows, dtype=torch.long)
        q_lat, q_rope, qpos = q_lat[rows], q_rope[rows], qpos[rows]
    if flavour == "bf16_eager":
        return attend_bf16_eager(q_lat, q_rope, k_lat, k_rope, sm_scale, mask=kpos <= qpos), None
    return attend(q_lat, q_rope, k_lat, k_rope, sm_scale, dtype, mask=kpos <= qpos)


def decode_flops(lengths, H: int, D: int, R: int) -> float:
    """Algorithmic flops of absorbed decode: ``2 H (2D + R)`` per cached token."""
    return float(2 * H * (2 * D + R) * np.sum(np.asarray(lengths, dtype=np.float64)))


def logsumexp_np(x) -> float:
    m = max(x)
    return m + math.log(sum(math.exp(v - m) for v in x))
