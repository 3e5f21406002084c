"""ctypes binding of libttfa.so (the C ABI declared in include/ttfa.h).

The library is loaded on first use.  If it is missing, every call raises
``LibraryNotBuilt``: there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libttfa.so"

TTFA_BF16 = 0
TTFA_F32 = 1
ABI_VERSION = 6

# Negative status codes of include/ttfa.h.
E_NULL, E_HEAD_DIM, E_GROUP, E_SEQ, E_ALIGN, E_DTYPE, E_SCALE, E_EPS, E_QROWS, E_SCRATCH = (
    -1, -2, -3, -4, -5, -6, -7, -8, -9, -10)
BWD_STATIC_MAX_ROWS = 1 << 20  # TTFA_BWD_STATIC_MAX_ROWS
EXPORTED = ("ttfa_abi_version", "ttfa_strerror", "ttfa_fwd", "ttfa_bwd", "ttfa_bwd_dq",
            "ttfa_bwd_dkdv", "ttfa_varlen_fwd", "ttfa_varlen_bwd", "ttfa_decode_workspace_bytes",
            "ttfa_decode_fwd", "ttfa_qk_prologue_fwd",
            "ttfa_qk_prologue_workspace_bytes", "ttfa_qk_prologue_bwd", "ttfa_bwd_static",
            "ttfa_d128_wide")


class LibraryNotBuilt(RuntimeError):
    pass


class TTFAError(RuntimeError):
    """A nonzero status from libttfa.so (``code`` < 0: argument error, > 0: hipError_t)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (ttfa status {code})")
        self.code = code


_lock = threading.Lock()
_lib = None

_vp, _i, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
_SIGS = {
    "ttfa_abi_version": ([], _i),
    "ttfa_strerror": ([_i], ctypes.c_char_p),
    "ttfa_fwd": ([_vp] * 5 + [_i] * 6 + [_f, _vp], _i),
    "ttfa_bwd": ([_vp] * 10 + [_i] * 6 + [_f, _vp], _i),
    "ttfa_bwd_dq": ([_vp] * 8 + [_i] * 6 + [_f, _vp], _i),
    "ttfa_bwd_dkdv": ([_vp] * 8 + [_i] * 6 + [_f, _vp], _i),
    "ttfa_varlen_fwd": ([_vp] * 6 + [_i] * 7 + [_f, _vp], _i),
    "ttfa_varlen_bwd": ([_vp] * 11 + [_i] * 7 + [_f, _vp], _i),
    "ttfa_decode_workspace_bytes": ([_i] * 6, ctypes.c_longlong),
    "ttfa_decode_fwd": ([_vp] * 7 + [_i] * 7 + [_f, _vp], _i),
    "ttfa_qk_prologue_fwd": ([_vp] * 12 + [_i] * 5 + [_f, _vp], _i),
    "ttfa_qk_prologue_workspace_bytes": ([_i] * 5, ctypes.c_longlong),
    "ttfa_qk_prologue_bwd": ([_vp] * 17 + [_i] * 5 + [_vp], _i),
    "ttfa_bwd_static": ([_vp] * 9 + [_i] * 6 + [_f, _vp], _i),
    "ttfa_d128_wide": ([_i] * 3 + [ctypes.POINTER(_i)] * 2, _i),
}


def d128_wide(B: int, Hq: int, T: int) -> tuple[bool, bool]:
    """(forward, dQ pass) of a bf16 D = 128 shape run the 256-row kernels (no HIP call)."""
    f, d = _i(), _i()
    check(load().ttfa_d128_wide(B, Hq, T, ctypes.byref(f), ctypes.byref(d)))
    return bool(f.value), bool(d.value)


def load() -> ctypes.CDLL:
    """Load (once) and return the library, with argument types declared."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise LibraryNotBuilt(
                    f"{LIB_PATH} is missing: build it with `python -m tinytrain_amd.build` "
                    "(the HIP library is the only implementation of these ops)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (argtypes, restype) in _SIGS.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = restype
            ver = lib.ttfa_abi_version()
            if ver != ABI_VERSION:
                raise LibraryNotBuilt(f"{LIB_PATH} has ABI {ver}, expected {ABI_VERSION}; rebuild it")
            _lib = lib
    return _lib


def strerror(code: int) -> str:
    return load().ttfa_strerror(code).decode()


def check(code: int) -> None:
    if code != 0:
        raise TTFAError(code, strerror(code))
