"""Oracle: byte layout of one packed INT2 cache row.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference fixes only the ABI around the packed row: 2-bit codes, four per
byte (``PF = 8 // bits``, ``MASK = 3``), ``D // group_size`` groups with FP32
``(scale, zero)`` each, one row per token slot
(``deployment/patches/rolaq_sglang.patch:26-34``,
``deployment/sglang/QuantKernel/mla_fused_writer.py:86-106``). The bit order
inside the row lives in an un-vendored SGLang fork, so this build defines it:

* A row of ``D`` codes is ``D / 16`` little-endian 32-bit words of 16 codes.
* Group ``g`` (``NG = D / 128`` groups) owns the words ``NG * s + g`` for
  ``s = 0 .. 7``; word ``s`` of group ``g`` holds the group's elements
  ``16 s .. 16 s + 15``.
* Element ``16 s + p`` sits at bits ``2p, 2p + 1`` of its word (LSB first).

Equivalently: the natural LSB-first packing of the row with its 32-bit words
reordered from (group, word) to (word, group). Every word holds one group
only, and the 16 bytes ``16 s .. 16 s + 15`` (D = 512) hold word ``s`` of all
four groups; the decode reader relies on both properties.

``params[slot, g] = (scale, zero)`` in FP32, i.e. ``[num_slots, NG, 2]``.
"""

from __future__ import annotations

import numpy as np

GROUP_SIZE = 128
CODES_PER_WORD = 16


def word_index(group: int, s: int, num_groups: int) -> int:
    """Index of word ``s`` of group ``group`` inside a row."""
    return num_groups * s + group


def element_position(j: np.ndarray | int, width: int):
    """Return ``(byte, bit)`` of row element ``j`` (vectorised)."""
    j = np.asarray(j)
    ng = width // GROUP_SIZE
    g = j // GROUP_SIZE
    f = j % GROUP_SIZE
    s = f // CODES_PER_WORD
    p = f % CODES_PER_WORD
    w = ng * s + g
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
    ng = width // GROUP_SIZE
    c = codes.astype(np.uint32).reshape(rows, ng, GROUP_SIZE // CODES_PER_WORD, CODES_PER_WORD)
    shifts = (2 * np.arange(CODES_PER_WORD, dtype=np.uint32))
    words_gs = (c << shifts).sum(axis=-1, dtype=np.uint64).astype(np.uint32)  # [rows, g, s]
    words = np.ascontiguousarray(words_gs.transpose(0, 2, 1)).reshape(rows, -1)  # [rows, s*ng+g]
    return words.astype("<u4").view(np.uint8).reshape(rows, width // 4)


def unpack_codes(packed: np.ndarray, width: int) -> np.ndarray:
    """Inverse of :func:`pack_codes`: ``[rows, D/4]`` bytes -> ``[rows, D]`` codes."""
    packed = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8))
    rows = packed.shape[0]
    if packed.shape[1] * 4 != width:
        raise ValueError("packed row length does not match the width")
    ng = width // GROUP_SIZE
    words = packed.view("<u4").reshape(rows, GROUP_SIZE // CODES_PER_WORD, ng)  # [rows, s, g]
    words = words.transpose(0, 2, 1)  # [rows, g, s]
    shifts = (2 * np.arange(CODES_PER_WORD, dtype=np.uint32))
    codes = (words[..., None].astype(np.uint32) >> shifts) & 3
    return codes.reshape(rows, width).astype(np.uint8)


def pack_codes_bitwise(codes: np.ndarray) -> np.ndarray:
    """Independent element-by-element packer used to pin :func:`pack_codes`."""
    codes = np.asarray(codes, dtype=np.uint8)
    rows, width = codes.shape
    out = np.zeros((rows, width // 4), dtype=np.uint8)
    for j in range(width):
        byte, bit = element_position(j, width)
        out[:, byte] |= (codes[:, j] & 3) << np.uint8(bit)
    return out
