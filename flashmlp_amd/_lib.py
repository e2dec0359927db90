"""ctypes binding of libflashmlp.so (the C ABI declared in include/flashmlp.h).

The library is loaded lazily, once. If it has not been built, every call raises: there
is no fallback path.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libflashmlp.so")

FMLP_OK = 0
FMLP_DTYPE_F16 = 0
FMLP_DTYPE_BF16 = 1
FMLP_DTYPE_F32 = 2
# OR-ed into the dtype code: outputs are fp32 arrays holding the unrounded fp32 sums
FMLP_OUT_F32 = 0x100
# OR-ed into the backward's dtype code: dW products with hi/lo io-dtype terms of h and dZ
FMLP_DW_HILO = 0x200
# OR-ed into the backward's dtype code: the recompute-only form (no stored dZ in the workspace)
FMLP_BWD_RECOMPUTE = 0x400
# OR-ed into the backward's dtype code: the stored-dZ form whenever the workspace allows (tests)
FMLP_BWD_STORE_DZ = 0x800
# OR-ed into the backward's dtype code: no dx wanted (dx may be NULL) / no dw1, dw2 wanted
FMLP_BWD_NO_DX = 0x1000
FMLP_BWD_NO_DW = 0x2000
ACT_CODES = {"": 0, "silu": 1, "leaky_relu": 2, "sigmoid": 3}

# (name, restype, argtypes) for every symbol include/flashmlp.h declares
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)
SIGNATURES = {
    "fmlp_abi_version": (ctypes.c_int, []),
    "fmlp_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "fmlp_last_error": (ctypes.c_char_p, []),
    "fmlp_act_from_name": (ctypes.c_int, [ctypes.c_char_p]),
    "fmlp_shape_supported": (ctypes.c_int, [_i64, _i64, _i64, _i64, ctypes.c_int]),
    "fmlp_shape_tuned": (ctypes.c_int, [_i64, _i64, ctypes.c_int]),
    "fmlp_fwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int, _vp]),
    "fmlp_fwd_strided": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64p, _i64p, _i64p,
                                        ctypes.c_int, ctypes.c_int, _vp]),
    "fmlp_fwd_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, ctypes.c_int]),
    "fmlp_fwd_ws": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int, _vp,
                                   ctypes.c_size_t, _vp]),
    "fmlp_bwd_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, ctypes.c_int]),
    "fmlp_bwd_stores_dz": (ctypes.c_int, [_i64, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int]),
    "fmlp_bwd_plan": (ctypes.c_int, [_i64, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int, _i64p, ctypes.c_int]),
    "fmlp_bwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_int,
                                ctypes.c_int, _vp, ctypes.c_size_t, _vp]),
    "fmlp_bwd_strided": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64p, _i64p,
                                        _i64p, _i64p, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_size_t, _vp]),
    "fmlp_bwd_noalloc": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_int,
                                        ctypes.c_int, _vp]),
}
FMLP_SCRATCH_MAX_BYTES = 64 << 20
ABI_VERSION = 4  # FMLP_ABI_VERSION of include/flashmlp.h

_lock = threading.Lock()
_lib = None


class FlashMLPLibraryError(RuntimeError):
    """libflashmlp.so is missing or does not match this package."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise FlashMLPLibraryError(
                    f"{LIB_PATH} is not built; run `python -m flashmlp_amd.build` (hipcc, gfx950)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            if handle.fmlp_abi_version() != ABI_VERSION:
                raise FlashMLPLibraryError("libflashmlp.so ABI version mismatch; rebuild it")
            _lib = handle
    return _lib


def strides(t) -> "ctypes.Array":
    """The three element strides of a 3-D tensor as an int64_t[3] for the *_strided calls."""
    return (ctypes.c_int64 * 3)(*t.stride())


def check(status: int, what: str) -> None:
    if status != FMLP_OK:
        L = lib()
        msg = L.fmlp_status_string(status).decode()
        detail = L.fmlp_last_error().decode()
        raise RuntimeError(f"flashmlp {what} failed: {msg}: {detail}")
