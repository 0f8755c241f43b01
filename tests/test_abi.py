"""C-ABI library: loads, exports every declared symbol, rejects bad arguments (CPU only)."""

import ctypes
import re
from pathlib import Path

import pytest

from mla_kv_quant_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "rolaq_mla.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|int)\s+(rolaq_\w+)\s*\(", text, re.M)))


def test_header_declares_the_entry_points():
    syms = declared_symbols()
    for name in ("rolaq_last_error", "rolaq_abi_version", "rolaq_scatter_pack_rows", "rolaq_write_rows",
                 "rolaq_norm_write_rows", "rolaq_prepare_gf_splits", "rolaq_decode_fwd", "rolaq_decode_partials", "rolaq_decode_merge", "rolaq_decode_split_cap", "rolaq_extend_fwd",
                 "rolaq_assemble_rows"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    # every declared symbol has a ctypes signature in the binding
    assert set(declared_symbols()) - {"rolaq_last_error"} <= set(_lib.SIGNATURES)
    assert lib.rolaq_abi_version() == 4


def test_invalid_arguments_are_rejected_before_any_launch():
    lib = _lib.load()
    assert lib.rolaq_prepare_gf_splits(None, None, None, 4, None) == _lib.ROLAQ_ERR_INVALID
    assert b"null pointer" in lib.rolaq_last_error()
    # n == 0 is a no-op even with null pointers
    assert lib.rolaq_prepare_gf_splits(None, None, None, 0, None) == _lib.ROLAQ_OK
    assert lib.rolaq_scatter_pack_rows(None, 512, None, 0, 512, 128, 0.98, 1.16, None, None, None) == 0
    bad = lib.rolaq_scatter_pack_rows(ctypes.c_void_p(16), 512, ctypes.c_void_p(16), 4, 384, 128,
                                      0.98, 1.16, ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert bad == _lib.ROLAQ_ERR_INVALID and b"D must be" in lib.rolaq_last_error()
    bad = lib.rolaq_scatter_pack_rows(ctypes.c_void_p(16), 512, ctypes.c_void_p(16), 4, 512, 64,
                                      0.98, 1.16, ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert bad == _lib.ROLAQ_ERR_INVALID and b"group_size" in lib.rolaq_last_error()
    bad = lib.rolaq_scatter_pack_rows(ctypes.c_void_p(16), 512, ctypes.c_void_p(16), 4, 512, 128,
                                      float("nan"), 1.16, ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert bad == _lib.ROLAQ_ERR_INVALID
    p = ctypes.c_void_p(256)
    args = [p, 16 * 576, 576, p, p, p, p, p, p, 3, p, p, 4, p, 8, 4, 16, 512, 64, 4, 16, 0.07, p, p, p, 8192, 512,
            None]
    assert lib.rolaq_decode_fwd(*args) == _lib.ROLAQ_ERR_INVALID  # page_size 3
    assert b"power of two" in lib.rolaq_last_error()
    args[9] = 1
    args[16] = 129  # more heads than the grid supports
    assert lib.rolaq_decode_fwd(*args) == _lib.ROLAQ_ERR_INVALID
    args[16] = 16
    args[12] = -1  # max_reqs
    assert lib.rolaq_decode_fwd(*args) == _lib.ROLAQ_ERR_INVALID and b"max_reqs" in lib.rolaq_last_error()
    args[12] = 4
    args[22] = ctypes.c_void_p(260)  # attn_logits must be 16-byte aligned
    assert lib.rolaq_decode_fwd(*args) == _lib.ROLAQ_ERR_INVALID and b"aligned" in lib.rolaq_last_error()
    args[22] = p
    # stage 1 alone takes the same arguments minus the output
    pargs = args[:22] + [p, p, None]
    pargs[9] = 3
    assert lib.rolaq_decode_partials(*pargs) == _lib.ROLAQ_ERR_INVALID
    assert b"decode_partials" in lib.rolaq_last_error()
    # stage 2 alone: D must be a cache width, pointers non-null
    assert lib.rolaq_decode_merge(p, p, p, 8, 4, 16, 384, p, 8192, 512, None) == _lib.ROLAQ_ERR_INVALID
    assert lib.rolaq_decode_merge(None, p, p, 8, 4, 16, 512, p, 8192, 512, None) == _lib.ROLAQ_ERR_INVALID
    assert lib.rolaq_decode_merge(None, None, None, 8, 0, 16, 512, None, 0, 0, None) == _lib.ROLAQ_OK
    # fused norm writer: rotation and norm weight are required, eps must be finite
    wargs = [p, 512, p, 1e-6, None, 0, p, 64, 1, p, p, p, None, p, 8, 512, 64, 4, 16, 8, 0.98, 1.16, p, p, p, p,
             p, p, None]
    assert lib.rolaq_norm_write_rows(*(wargs[:14] + [0] + wargs[15:])) == _lib.ROLAQ_OK  # n == 0
    bad = list(wargs)
    bad[9] = None
    assert lib.rolaq_norm_write_rows(*bad) == _lib.ROLAQ_ERR_INVALID and b"rotation_t" in lib.rolaq_last_error()
    bad = list(wargs)
    bad[2] = None
    assert lib.rolaq_norm_write_rows(*bad) == _lib.ROLAQ_ERR_INVALID and b"norm_weight" in lib.rolaq_last_error()
    bad = list(wargs)
    bad[3] = float("inf")
    assert lib.rolaq_norm_write_rows(*bad) == _lib.ROLAQ_ERR_INVALID and b"eps" in lib.rolaq_last_error()
    bad = list(wargs)
    bad[4], bad[5] = p, 100
    assert lib.rolaq_norm_write_rows(*bad) == _lib.ROLAQ_ERR_INVALID and b"latent_out" in lib.rolaq_last_error()
    bad = list(wargs)
    bad[15] = 384
    assert lib.rolaq_norm_write_rows(*bad) == _lib.ROLAQ_ERR_INVALID and b"(D, R)" in lib.rolaq_last_error()
    # extend: shape and pointer checks, empty batch is a no-op
    eargs = [p, 40 * 288, 288, p, 288, p, p, p, 16, p, p, 4, p, p, p, p, 4, 40, 256, 32, 4, 16, 2048, 0.1, p, 1,
             1, p, 40 * 256, 256, None]
    bad = list(eargs)
    bad[18], bad[19] = 384, 32
    assert lib.rolaq_extend_fwd(*bad) == _lib.ROLAQ_ERR_INVALID and b"(D, R)" in lib.rolaq_last_error()
    bad = list(eargs)
    bad[8] = 12
    assert lib.rolaq_extend_fwd(*bad) == _lib.ROLAQ_ERR_INVALID and b"power of two" in lib.rolaq_last_error()
    bad = list(eargs)
    bad[3] = None
    assert lib.rolaq_extend_fwd(*bad) == _lib.ROLAQ_ERR_INVALID
    bad = list(eargs)
    bad[11] = -2
    assert lib.rolaq_extend_fwd(*bad) == _lib.ROLAQ_ERR_INVALID and b"max_reqs" in lib.rolaq_last_error()
    bad = list(eargs)
    bad[24] = None
    assert lib.rolaq_extend_fwd(*bad) == _lib.ROLAQ_ERR_INVALID and b"null" in lib.rolaq_last_error()
    bad = list(eargs)
    bad[25] = 0
    assert lib.rolaq_extend_fwd(*bad) == _lib.ROLAQ_ERR_INVALID and b"workspace" in lib.rolaq_last_error()
    bad = list(eargs)
    bad[26] = 2  # more key rows than the workspace holds
    assert lib.rolaq_extend_fwd(*bad) == _lib.ROLAQ_ERR_INVALID and b"short" in lib.rolaq_last_error()
    bad = list(eargs)
    bad[26] = -1
    assert lib.rolaq_extend_fwd(*bad) == _lib.ROLAQ_ERR_INVALID
    # decode split cap: argument checks (a valid call reads the device's CU count)
    cap = ctypes.c_int(-7)
    assert lib.rolaq_decode_split_cap(0, 16, 512, 129, ctypes.byref(cap)) == _lib.ROLAQ_ERR_INVALID
    assert lib.rolaq_decode_split_cap(32, 16, 384, 129, ctypes.byref(cap)) == _lib.ROLAQ_ERR_INVALID
    assert lib.rolaq_decode_split_cap(32, 16, 512, 129, None) == _lib.ROLAQ_ERR_INVALID
    assert cap.value == -7
    bad = list(eargs)
    bad[16] = 0
    assert lib.rolaq_extend_fwd(*bad) == _lib.ROLAQ_OK
    # assemble: shapes, strides, pointers; n == 0 is a no-op
    aargs = [p, 10, p, p, p, p, p, p, None, 512, 64, p, 576, None]
    bad = list(aargs)
    bad[9], bad[10] = 512, 32
    assert lib.rolaq_assemble_rows(*bad) == _lib.ROLAQ_ERR_INVALID and b"(D, R)" in lib.rolaq_last_error()
    bad = list(aargs)
    bad[12] = 500
    assert lib.rolaq_assemble_rows(*bad) == _lib.ROLAQ_ERR_INVALID and b"stride" in lib.rolaq_last_error()
    bad = list(aargs)
    bad[0] = None
    assert lib.rolaq_assemble_rows(*bad) == _lib.ROLAQ_ERR_INVALID
    bad = list(aargs)
    bad[1] = 0
    assert lib.rolaq_assemble_rows(*bad) == _lib.ROLAQ_OK


def test_check_raises_value_error():
    lib = _lib.load()
    rc = lib.rolaq_prepare_gf_splits(None, None, None, 4, None)
    with pytest.raises(ValueError):
        _lib.check(rc)


def test_pool_memory_accounting_matches_its_buffers():
    """get_kv_size_bytes charges per-token rows of every layer, the shared row
    map once, and the fixed BF16 window arena (rolaq_sglang.patch:166-189)."""
    import torch
    from mla_kv_quant_amd import PackedMLAPool

    for D, R, layers, reqs in ((512, 64, 3, 5), (256, 32, 2, 9)):
        pool = PackedMLAPool(300, layers, D, R, reqs, 4, 16, device="cpu")
        held = sum(t.numel() * t.element_size() for name in ("c_codes", "c_params", "rope_buf", "hp_c")
                   for t in getattr(pool, name))
        held += pool.hp_row_of_slot.numel() * 4 + pool.hp_owner_of_row.numel() * 4
        assert pool.get_kv_size_bytes() == held
        per_token = layers * (D // 4 + 8 * (D // 128) + 2 * R) + 4
        assert per_token == (layers * 288 + 4 if D == 512 else layers * 144 + 4)
