"""Oracle: byte layout of one packed INT2 cache row.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference fixes only the ABI around the packed row: 2-bit codes, four per
byte (``PF = 8 // bits``, ``MASK = 3``), ``D // group_size`` groups with FP32
``(scale, zero)`` each, one row per token slot
(``deployment/patches/rolaq_sglang.patch:26-34``,
``deployment/sglang/QuantKernel/mla_fused_writer.py:86-106``). The bit order
inside the row lives in an un-vendored SGLang fork, so this build defines it
as the natural LSB-first packing:

* element ``j`` of the row sits at byte ``j >> 2``, bits ``2 (j & 3)`` and
  ``2 (j & 3) + 1``;
* equivalently, the row is ``D / 16`` little-endian 32-bit words of 16 codes,
  group ``g`` (``NG = D / 128``) owns the eight consecutive words
  ``8 g .. 8 g + 7`` (32 bytes), word ``8 g + s`` holds the group's elements
  ``16 s .. 16 s + 15`` with element ``16 s + p`` at bits ``2p, 2p + 1``.

Every word holds one group only, and one group's codes are 32 contiguous
bytes; the decode reader relies on both properties (a lane loads its group's
32 bytes with two 16-byte loads and applies one ``(scale, zero)`` to them).

``params[slot, g] = (scale, zero)`` in FP32, i.e. ``[num_slots, NG, 2]``.
"""

from __future__ import annotations

import numpy as np

GROUP_SIZE = 128
CODES_PER_WORD = 16
WORDS_PER_GROUP = GROUP_SIZE // CODES_PER_WORD


def word_index(group: int, s: int) -> int:
    """Index of word ``s`` of group ``group`` inside a row."""
    return WORDS_PER_GROUP * group + s


def element_position(j: np.ndarray | int, width: int):
    """Return ``(byte, bit)`` of row element ``j`` (vectorised), computed
    through the (group, word, code) decomposition."""
    j = np.asarray(j)
    g = j // GROUP_SIZE
    f = j % GROUP_SIZE
    s = f // CODES_PER_WORD
    p = f % CODES_PER_WORD
    w = word_index(g, s)
    return 4 * w + p // 4, 2 * (p % 4)


def pack_codes(codes: np.ndarray) -> np.ndarray:
    """Pack ``codes`` (uint8 in 0..3, shape ``[rows, D]``) into ``[rows, D/4]`` bytes."""
    codes = np.asarray(codes)
    if codes.ndim != 2:
        raise ValueError("codes must be [rows, D]")
    rows, width = codes.shape
    if width % GROUP_SIZE:
        raise ValueError("width must be a multiple of 128")
    if codes.size and int(codes.max()) > 3:
        raise ValueError("codes must be 2-bit")
    c = codes.astype(np.uint8).reshape(rows, width // 4, 4)
    shifts = (2 * np.arange(4, dtype=np.uint8))
    return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint8)


def unpack_codes(packed: np.ndarray, width: int) -> np.ndarray:
    """Inverse of :func:`pack_codes`: ``[rows, D/4]`` bytes -> ``[rows, D]`` codes."""
    packed = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8))
    rows = packed.shape[0]
    if packed.shape[1] * 4 != width:
        raise ValueError("packed row length does not match the width")
    shifts = (2 * np.arange(4, dtype=np.uint8))
    codes = (packed[..., None] >> shifts) & 3
    return codes.reshape(rows, width).astype(np.uint8)


def pack_codes_bitwise(codes: np.ndarray) -> np.ndarray:
    """Independent element-by-element packer used to pin :func:`pack_codes`:
    goes through :func:`element_position` (group / word / code) one element at
    a time."""
    codes = np.asarray(codes, dtype=np.uint8)
    rows, width = codes.shape
    out = np.zeros((rows, width // 4), dtype=np.uint8)
    for j in range(width):
        byte, bit = element_position(j, width)
        out[:, byte] |= (codes[:, j] & 3) << np.uint8(bit)
    return out
