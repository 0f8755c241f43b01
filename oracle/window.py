"""Oracle: the s4r16 BF16 window and the cache writer's stores.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates
* ``mla_quant/cache.py:775-800`` (``_target_window_state``: 0 pad, 1 BF16,
  2 quantized; sink = first P valid rows, recent = last W valid rows);
* ``deployment/sglang/QuantKernel/mla_fused_writer.py:36-51`` (``_aux``: keep
  mask, ring row, rope/window/ownership stores);
* ``mla_fused_writer.py:110-224`` + ``rolaq_sglang.patch:9-34,155-164``
  (what one writer call leaves in the pool).
"""

from __future__ import annotations

import numpy as np
import torch

from . import codec, layout


def ring_row(req, pos, P: int, W: int):
    """mla_fused_writer.py:43 -- ring row of position ``pos`` of request ``req``."""
    req = np.asarray(req, dtype=np.int64)
    pos = np.asarray(pos, dtype=np.int64)
    inner = np.where(pos < P, pos, P + np.maximum(pos - P, 0) % max(W, 1))
    return 1 + req * (P + W) + inner


def keep_mask(pos, seq, req, slot, P: int, W: int, max_reqs: int):
    """mla_fused_writer.py:41 -- which rows claim a ring row (slot 0 never does)."""
    pos = np.asarray(pos, dtype=np.int64)
    seq = np.asarray(seq, dtype=np.int64)
    req = np.asarray(req, dtype=np.int64)
    slot = np.asarray(slot, dtype=np.int64)
    return ((pos < P) | (pos >= seq - W)) & (req < max_reqs) & (req >= 0) & (slot > 0)


def target_window_state(valid: torch.Tensor, sink: int, recent: int) -> torch.Tensor:
    """cache.py:775-800 -- per-row state after an append (padding-aware)."""
    valid = valid.to(torch.bool)
    state = valid.to(torch.uint8) * 2
    if sink:
        from_start = valid.to(torch.int64).cumsum(dim=-1)
        s = valid & (from_start <= sink)
    else:
        s = torch.zeros_like(valid)
    if recent:
        from_end = valid.flip(-1).to(torch.int64).cumsum(dim=-1).flip(-1)
        r = valid & (from_end <= recent)
    else:
        r = torch.zeros_like(valid)
    state.masked_fill_(s | r, 1)
    return state


def positional_bf16(pos, length: int, P: int, W: int):
    """Read-side rule for an unpadded sequence of ``length`` tokens: position
    ``pos`` is served from the BF16 window iff it is one of the first ``P`` or
    last ``W`` tokens (``target_window_state`` with every row valid)."""
    pos = np.asarray(pos, dtype=np.int64)
    return (pos < P) | (pos >= length - W)


def write_rows(pool: dict, x: torch.Tensor, k_pe: torch.Tensor, loc, seq, req,
               rotation: torch.Tensor | None, threshold: float, gain: float,
               P: int, W: int, max_reqs: int, positions=None) -> torch.Tensor:
    """Apply one writer call to a numpy ``pool`` dict in place.

    ``pool`` holds ``codes`` uint8 ``[slots, D/4]``, ``params`` float32
    ``[slots, NG, 2]``, ``rope`` uint16 (bf16 bits) ``[slots, R]``, ``hp`` uint16
    ``[rows, D]``, ``row_of_slot`` int32 ``[slots]``, ``owner_of_row`` int32.
    ``x`` is the un-rotated latent (bf16 ``[n, D]``), ``k_pe`` bf16 ``[n, R]``.
    ``positions`` defaults to ``seq - 1`` (a decode step, mla_fused_writer.py:40).
    Returns the FP32 rotated rows the codec saw.
    """
    loc = np.asarray(loc, dtype=np.int64)
    seq = np.asarray(seq, dtype=np.int64)
    req = np.asarray(req, dtype=np.int64)
    pos = seq - 1 if positions is None else np.asarray(positions, dtype=np.int64)
    n, width = x.shape
    # mla_fused_writer.py:142-149: FP32 GEMM with R_eff = fp32(bf16(R)).
    c = codec.rotate(x, rotation) if rotation is not None else x.float()
    codes, scale, zero, _ = codec.lloyd_codec(c, codec.GROUP_SIZE, threshold, codec.snap_gain(gain))
    packed = layout.pack_codes(codes.numpy())
    pool["codes"][loc] = packed
    pool["params"][loc, :, 0] = scale.numpy()
    pool["params"][loc, :, 1] = zero.numpy()
    keep = keep_mask(pos, seq, req, loc, P, W, max_reqs)
    ring = ring_row(req, pos, P, W)
    live = loc > 0
    pe_bits = k_pe.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)
    pool["rope"][loc[live]] = pe_bits[live]
    c_bits = c.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)
    pool["hp"][ring[keep]] = c_bits[keep]
    pool["owner_of_row"][ring[keep]] = loc[keep].astype(np.int32)
    pool["row_of_slot"][loc[live]] = np.where(keep[live], ring[live], -1).astype(np.int32)
    return c


def new_pool(num_slots: int, D: int, R: int, max_reqs: int, P: int, W: int) -> dict:
    """Zeroed numpy pool arrays with the reference's shapes (one layer)."""
    ng = D // codec.GROUP_SIZE
    hp_rows = 1 + max_reqs * (P + W)
    return {
        "codes": np.zeros((num_slots, D // 4), np.uint8),
        "params": np.zeros((num_slots, ng, 2), np.float32),
        "rope": np.zeros((num_slots, R), np.uint16),
        "hp": np.zeros((hp_rows, D), np.uint16),
        "row_of_slot": np.full((num_slots,), -1, np.int32),
        "owner_of_row": np.zeros((hp_rows,), np.int32),
    }
