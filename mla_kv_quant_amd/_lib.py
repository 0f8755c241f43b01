"""ctypes binding of ``librolaq_mla.so`` (declared in ``include/rolaq_mla.h``).

The library is built in-tree by ``mla_kv_quant_amd.build``. There is no
fallback: if the library is missing or a symbol is absent, loading raises.
"""

from __future__ import annotations

import ctypes
from ctypes import c_double, c_float, c_int, c_int64, c_void_p, c_char_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "librolaq_mla.so"

ROLAQ_OK = 0
ROLAQ_ERR_INVALID = 1
ROLAQ_ERR_HIP = 2

# symbol -> argtypes (all return int except rolaq_last_error)
SIGNATURES = {
    "rolaq_abi_version": [],
    "rolaq_scatter_pack_rows": [c_void_p, c_int64, c_void_p, c_int64, c_int, c_int, c_float, c_double,
                                c_void_p, c_void_p, c_void_p],
    "rolaq_write_rows": [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
                         c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int, c_int, c_float,
                         c_double, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                         c_void_p],
    "rolaq_norm_write_rows": [c_void_p, c_int64, c_void_p, c_float, c_void_p, c_int64, c_void_p, c_int64,
                              c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int,
                              c_int, c_int, c_int, c_float, c_double, c_void_p, c_void_p, c_void_p, c_void_p,
                              c_void_p, c_void_p, c_void_p],
    "rolaq_prepare_gf_splits": [c_void_p, c_void_p, c_void_p, c_int64, c_void_p],
    "rolaq_decode_fwd": [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                         c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int,
                         c_int, c_int, c_int, c_float, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
                         c_void_p],
    "rolaq_decode_fwd_noalloc": [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                 c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int,
                                 c_int, c_int, c_int, c_float, c_void_p, c_int64, c_int64, c_void_p],
    "rolaq_decode_partials": [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                              c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int,
                              c_int, c_int, c_int, c_float, c_void_p, c_void_p, c_void_p],
    "rolaq_decode_split_cap": [c_int, c_int, c_int, c_int, c_void_p],
    "rolaq_decode_merge": [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_int64,
                           c_int64, c_void_p],
    "rolaq_extend_fwd": [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int,
                         c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                         c_int, c_int, c_int, c_int, c_float, c_void_p, c_int64, c_int64, c_void_p, c_int64,
                         c_int64, c_void_p],
    "rolaq_assemble_rows": [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                            c_void_p, c_int, c_int, c_void_p, c_int64, c_void_p],
}

_LIB: ctypes.CDLL | None = None


class RolaqError(RuntimeError):
    """Raised when a C-ABI call returns a non-zero status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"rolaq error {code}: {message}")
        self.code = code


def load() -> ctypes.CDLL:
    """Load the library once; raise if it is missing or incomplete."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m mla_kv_quant_amd.build` "
            "(there is no CPU fallback for the packed-INT2 path)")
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.rolaq_last_error.restype = c_char_p
    lib.rolaq_last_error.argtypes = []
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = c_int
        fn.argtypes = args
    _LIB = lib
    return lib


def check(rc: int) -> None:
    if rc != ROLAQ_OK:
        msg = load().rolaq_last_error().decode(errors="replace")
        if rc == ROLAQ_ERR_INVALID:
            raise ValueError(msg)
        raise RolaqError(rc, msg)
