"""ctypes binding of ``libknlp_int4kv.so`` (C ABI in include/knlp_int4kv.h).

The library is loaded from the package directory only.  A missing library is
an error, never a silent fallback: every operator in :mod:`knlp_amd.ops`
calls :func:`lib` and raises when the HIP path is unavailable.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libknlp_int4kv.so")
ABI_VERSION = 1

# enum knlp_status
OK, ERR_SHAPE, ERR_DTYPE, ERR_ALIGN, ERR_WORKSPACE, ERR_LAUNCH, ERR_ARG = 0, -1, -2, -3, -4, -5, -6
# enum knlp_dtype
DT_F16, DT_BF16, DT_I32, DT_I64 = 0, 1, 2, 3
# enum knlp_kv_format
KV_INT4_SYM, KV_INT4_ASYM, KV_INT8_SYM, KV_FP16 = 0, 1, 2, 3

EXPORTS = (
    "knlp_abi_version", "knlp_status_string", "knlp_kv_append",
    "knlp_kv_decode_split_tokens", "knlp_kv_decode_plan", "knlp_kv_decode_workspace_bytes",
    "knlp_kv_decode_partial", "knlp_kv_decode_merge", "knlp_kv_decode",
    "knlp_kv_decode_kernel_kind", "knlp_kv_append_decode", "knlp_int4_twos_to_offset",
    "knlp_kv_decode_noalloc", "knlp_hbm_read_probe",
)


class KvPlane(ctypes.Structure):
    """``struct knlp_kv_plane``."""
    _fields_ = [
        ("data", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("zeros", ctypes.c_void_p),
        ("stride_block", ctypes.c_int64), ("stride_page", ctypes.c_int64),
        ("stride_head", ctypes.c_int64),
        ("s_stride_block", ctypes.c_int64), ("s_stride_page", ctypes.c_int64),
        ("s_stride_head", ctypes.c_int64),
        ("z_stride_block", ctypes.c_int64), ("z_stride_page", ctypes.c_int64),
        ("z_stride_head", ctypes.c_int64),
        ("format", ctypes.c_int32), ("group_size", ctypes.c_int32),
    ]


_lock = threading.Lock()
_lib = None

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float
_PLANE = ctypes.POINTER(KvPlane)

_SIGS = {
    "knlp_abi_version": (_I32, []),
    "knlp_status_string": (ctypes.c_char_p, [_I32]),
    "knlp_kv_append": (_I32, [_P, _P, _I32, _I64, _I32, _I32, _I64, _I64, _I64, _I64,
                              _PLANE, _PLANE, _P, _I32, _I32, _F, _P]),
    "knlp_kv_decode_split_tokens": (_I32, [_I32, _I32, _I32, _I32, _I32, _I32, _I32]),
    "knlp_kv_decode_plan": (_I32, [_I32, _I32, _I32, _I32, _I32, _I64, _I32, _I32, _I32, _I32]),
    "knlp_kv_decode_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32, _I32]),
    "knlp_kv_decode_partial": (_I32, [_P, _I32, _I64, _I64, _I32, _I32, _I32, _I32,
                                      _PLANE, _PLANE, _P, _I64, _P, _I32, _I32, _F, _I32,
                                      _P, _I64, _P]),
    "knlp_kv_decode_merge": (_I32, [_P, _I64, _P, _I32, _I32, _I32, _I32, _I32, _P, _I32,
                                    _I64, _I64, _P]),
    "knlp_kv_decode": (_I32, [_P, _I32, _I64, _I64, _I32, _I32, _I32, _I32, _PLANE, _PLANE,
                              _P, _I64, _P, _I32, _I32, _F, _I32, _P, _I64, _P, _I32, _I64,
                              _I64, _P]),
    "knlp_kv_decode_noalloc": (_I32, [_P, _I32, _I64, _I64, _I32, _I32, _I32, _I32, _PLANE,
                                      _PLANE, _P, _I64, _P, _I32, _I32, _F, _I32, _P, _I32,
                                      _I64, _I64, _P]),
    "knlp_kv_decode_kernel_kind": (_I32, [_I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32]),
    "knlp_hbm_read_probe": (_I32, [_P, _I64, _P, _I32, _P]),
    "knlp_int4_twos_to_offset": (_I32, [_P, _I64, _P, _I64, _I64, _I64, _P]),
    "knlp_kv_append_decode": (_I32, [_P, _I32, _I64, _I64, _I32, _I32, _I32, _I32,
                                     _P, _P, _I32, _I64, _I64, _I64, _I64, _P, _I32, _F,
                                     _PLANE, _PLANE, _P, _I64, _P, _I32, _I32, _F, _I32, _P,
                                     _I64, _P, _I32, _I64, _I64, _P]),
}


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"knlp_amd HIP library not built: {LIB_PATH} is missing "
                    "(run `python -m knlp_amd.build`); there is no CPU fallback")
            h = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(h, name)
                fn.restype = res
                fn.argtypes = args
            v = h.knlp_abi_version()
            if v != ABI_VERSION:
                raise RuntimeError(f"knlp_amd ABI mismatch: library {v}, bindings {ABI_VERSION}")
            _lib = h
    return _lib


def check(status: int, what: str) -> None:
    """Turn a negative status into the Python exception the reference raises
    for the same misuse (ValueError for shapes / dtypes / arguments)."""
    if status >= 0:
        return
    msg = lib().knlp_status_string(status).decode()
    if status == ERR_LAUNCH:
        raise RuntimeError(f"{what}: {msg}")
    raise ValueError(f"{what}: {msg} (status {status})")
