"""ctypes loader for ``libgdn_kernel_amd.so`` (the C ABI in include/gdn_kernel_amd.h).

The library is built in-tree by ``gdn_kernel_amd.build``.  There is no fallback
implementation: if the shared object is missing or fails to load, every entry
point raises.
"""
from __future__ import annotations

import ctypes
from ctypes import c_double, c_int, c_int32, c_int64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libgdn_kernel_amd.so"

GDN_OK = 0
GDN_ERR_INVALID_ARGUMENT = 1
GDN_ERR_UNSUPPORTED = 2
GDN_ERR_DEVICE = 3
GDN_INDEX_INT32 = 0
GDN_INDEX_INT64 = 1
GDN_MAX_HEADS = 65536
GDN_PREFILL_NO_ALLOC_SCRATCH_BYTES = 64 << 20
GDN_PREFILL_DROPIN_SCRATCH_BYTES = 128 << 20
GDN_PREFILL_DROPIN_TWO_KERNEL_TOKENS = 1024

# Exported symbols and their argument types (must match include/gdn_kernel_amd.h and
# include/gdn_kernel_amd_testing.h).
_P = c_void_p
_HEADS = [c_int32, c_int32, c_int32, c_int32, c_int32]
SIGNATURES = {
    "gdn_version": ([], c_int),
    "gdn_last_error": ([], ctypes.c_char_p),
    "gdn_build_id": ([], ctypes.c_char_p),
    "gdn_decode": ([_P] * 8 + [c_double, _P, _P, c_int64] + _HEADS + [_P], c_int),
    "gdn_decode_check": ([_P] * 8 + [c_double, _P, _P, c_int64] + _HEADS, c_int),
    "gdn_decode_pooled": ([_P, _P, _P, _P, c_int64, _P, _P, _P, _P, _P, c_double, _P, c_int64]
                          + _HEADS + [_P], c_int),
    "gdn_decode_pooled_check": ([_P, _P, _P, _P, c_int64, _P, _P, _P, _P, _P, c_double, _P,
                                 c_int64] + _HEADS, c_int),
    "gdn_prefill": ([_P] * 8 + [_P, c_int32, c_int64, c_int64, c_double, _P, _P] + _HEADS + [_P],
                    c_int),
    "gdn_prefill_check": ([_P] * 8 + [_P, c_int32, c_int64, c_int64, c_double, _P, _P] + _HEADS,
                          c_int),
    "gdn_prefill_workspace_size": ([c_int64, c_int64, c_int32], c_int64),
    "gdn_prefill_with_workspace": ([_P] * 8 + [_P, c_int32, c_int64, c_int64, c_double, _P, _P]
                                   + _HEADS + [_P, c_int64, _P], c_int),
    "gdn_prefill_giveups": ([ctypes.POINTER(ctypes.c_uint64), c_int32], c_int),
    "gdn_decode_pool_conflicts": ([ctypes.POINTER(ctypes.c_uint64), c_int32], c_int),
    "gdn_static_device_bytes": ([], c_int64),
    "gdn_prefill_no_alloc": ([_P] * 8 + [_P, c_int32, c_int64, c_int64, c_double, _P, _P] + _HEADS
                             + [_P], c_int),
    # include/gdn_kernel_amd_testing.h
    "gdn_decode_num_variants": ([], c_int),
    "gdn_decode_with_variant": ([_P] * 8 + [c_double, _P, _P, c_int64] + _HEADS + [c_int32, _P], c_int),
    "gdn_decode_pooled_with_variant": ([_P, _P, _P, _P, c_int64, _P, _P, _P, _P, _P, c_double, _P,
                                        c_int64] + _HEADS + [c_int32, _P], c_int),
    "gdn_prefill_fault_injection": ([_P] * 8 + [_P, c_int32, c_int64, c_int64, c_double, _P, _P]
                                    + _HEADS + [c_int32, c_int32, _P, _P], c_int),
}

_lib = None


class GDNError(RuntimeError):
    """A failure reported by the C ABI (device or launch error)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[gdn error {code}] {message}")
        self.code = code


def load() -> ctypes.CDLL:
    """Load (once) and return the shared library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH.name} is not built; run `python -m gdn_kernel_amd.build` "
            "(there is no non-HIP fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    _lib = lib
    return lib


def last_error() -> str:
    return load().gdn_last_error().decode()


def check(rc: int) -> None:
    """Map a C-ABI status to a Python exception."""
    if rc == GDN_OK:
        return
    msg = last_error()
    if rc in (GDN_ERR_INVALID_ARGUMENT, GDN_ERR_UNSUPPORTED):
        raise ValueError(f"[gdn error {rc}] {msg}")
    raise GDNError(rc, msg)
