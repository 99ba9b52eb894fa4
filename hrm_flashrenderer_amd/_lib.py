"""ctypes binding of libfa_mi355x.so (C ABI: include/fa_mi355x.h).

`torch` is imported before the library is opened so that the library's
DT_NEEDED libamdhip64.so.7 resolves to the HIP runtime torch already loaded:
one runtime per process, shared streams.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded before the HIP library, see above)

from ._build import LIB_PATH

FA_ABI_VERSION = 4
FA_DTYPE_F16 = 0
FA_DTYPE_F32 = 1

# (name, restype, argtypes) of every exported symbol, in header order.
_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
SYMBOLS = (
    ("fa_flash_attn_fwd", _I,
     [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I64, _I64, _P, _P, _P]),
    ("fa_flash_attn_fwd_ws", _I,
     [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I64, _I64, _P, _P, _P, _SZ, _P]),
    ("fa_flash_attn_workspace_bytes", _SZ, [_I, _I, _I, _I, _I, _I, _I]),
    ("fa_flash_attn_paged_fwd", _I,
     [_P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I64, _I64, _P, _P, _P, _P,
      _I, _I, _P, _SZ, _P]),
    ("fa_flash_attn_paged_fwd_noalloc", _I,
     [_P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I64, _I64, _P, _P, _P, _P,
      _I, _I, _P]),
    ("fa_paged_workspace_bytes", _SZ, [_I, _I, _I, _I, _I, _I, _I, _I]),
    ("fa_paged_kv_append", _I,
     [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I64, _P, _P, _I, _P]),
    ("fa_flash_attn_paged_rope_fwd", _I,
     [_P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I64, _I64, _P, _P, _P, _P,
      _I, _I, _P, _SZ, _P, _P, _I, _P]),
    ("fa_paged_kv_append_rope", _I,
     [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I64, _P, _P, _I, _P, _P, _I, _P]),
    ("fa_paged_kv_scatter", _I,
     [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _I, _P]),
    ("fa_flash_attn_paged_append_fwd", _I,
     [_P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I64, _P, _P, _I, _I, _P, _P, _I,
      _I64, _P, _P, _P, _I, _P, _SZ, _P]),
    ("fa_decode_token_major", _I,
     [_P, _P, _P, _P, _I, _I, _I, _I, ctypes.c_float, _P, _I, _P, _SZ, _P]),
    ("fa_decode_token_major_workspace_bytes", _SZ, [_I, _I, _I, _I, _I]),
    ("fa_last_error", ctypes.c_char_p, []),
    ("fa_abi_version", _I, []),
)

_lock = threading.Lock()
_lib = None


class LibraryMissing(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Open the built library (once). Raises LibraryMissing if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is not built; run `python -m hrm_flashrenderer_amd._build` "
                "(or __graft_entry__.build())")
        lib = ctypes.CDLL(LIB_PATH)
        for name, restype, argtypes in SYMBOLS:
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        ver = lib.fa_abi_version()
        if ver != FA_ABI_VERSION:
            raise RuntimeError(f"libfa_mi355x ABI {ver}, expected {FA_ABI_VERSION}")
        _lib = lib
    return _lib


def check(status: int) -> None:
    """Raise RuntimeError with the library's message on a non-zero status."""
    if status != 0:
        msg = load().fa_last_error().decode("utf-8", "replace")
        raise RuntimeError(msg or f"libfa_mi355x error {status}")
