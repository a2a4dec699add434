"""ctypes binding of libomni_int8.so (the C ABI declared in include/omni_int8.h).

The shared library is built in-tree by ``make -C omni-rs_amd`` (or
``__graft_entry__.build()``). There is no fallback: if the library is missing
or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import os

OMNI_OK = 0
OMNI_NOT_HANDLED = 1
OMNI_NO_DEVICE = 2
OMNI_BAD_ARGUMENT = 3
OMNI_HIP_ERROR = -1

OMNI_F32 = 0
OMNI_F16 = 1

OMNI_LOWERING_AUTO = 0
OMNI_LOWERING_MFMA = 1
OMNI_LOWERING_SCALAR = 2

# OMNI_INT8_LIBRARY may name another build of the same library (the
# host-sanitised one that tests/sanitize_cpu.sh runs the CPU tests on).
LIB_PATH = os.environ.get("OMNI_INT8_LIBRARY") or os.path.join(
    os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "libomni_int8.so")

# name -> (restype, argtypes); one entry per declaration in include/omni_int8.h
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
SIGNATURES = {
    "omni_int8_arch_supported": (_INT, [_INT]),
    "omni_w8a8_lowering": (_INT, [_I64]),
    "omni_int8_last_error": (ctypes.c_char_p, []),
    "omni_int8_set_tuning": (_INT, [ctypes.c_char_p, _INT, _INT]),
    "omni_int8_quantize_rows": (_INT, [_P, _INT, _I64, _I64, _I64, _P, _P, _P, _P]),
    "omni_w8a8_gemm": (_INT, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _INT, _P, _INT, _P]),
    "omni_w8a8_gemm_workspace_size": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "omni_w8a8_gemm_ws": (_INT, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _INT, _P, _INT, _P,
                                 ctypes.c_size_t, _P]),
    "omni_try_int8_gemm_workspace_size": (ctypes.c_size_t, [_I64, _I64]),
    "omni_try_int8_gemm_split_workspace_size": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "omni_try_int8_gemm": (_INT, [_P, _INT, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _P,
                                  ctypes.c_size_t, _P]),
    "omni_try_int8_gemm_noalloc": (_INT, [_P, _INT, _I64, _I64, _P, _I64, _P, _I64, _P, _I64,
                                          _P, _P]),
    "omni_w8a16_gemm": (_INT, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _P]),
    "omni_w8a16_gemm_workspace_size": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "omni_w8a16_gemm_ws": (_INT, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, ctypes.c_size_t, _P]),
    "omni_w4a16_gemm": (_INT, [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _P]),
    "omni_w4a16_gemm_workspace_size": (ctypes.c_size_t, [_I64, _I64, _I64, _I64]),
    "omni_w4a16_gemm_ws": (_INT, [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _P, ctypes.c_size_t, _P]),
    "omni_f16_gemv": (_INT, [_P, _P, _I64, _I64, _I64, _P, _P]),
    "omni_f16_gemm": (_INT, [_P, _P, _I64, _I64, _I64, _P, _P]),
    "omni_convrot_quantize_rows": (_INT, [_P, _INT, _I64, _I64, _I64, _I64, _P, _P, _P, _P]),
    "omni_convrot_linear": (_INT, [_P, _INT, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _INT,
                                   _P, ctypes.c_size_t, _P]),
}

_lib = None


class OmniError(RuntimeError):
    """A non-OK status from libomni_int8 (other than the reference's None)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"libomni_int8 status {status}: {message}")
        self.status = status


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OmniError(OMNI_BAD_ARGUMENT,
                            f"{LIB_PATH} is missing; build it with `make -C omni-rs_amd`")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().omni_int8_last_error().decode(errors="replace")


def check(status: int) -> int:
    """Raise on anything but OK / NOT_HANDLED; return the status."""
    if status not in (OMNI_OK, OMNI_NOT_HANDLED):
        raise OmniError(status, last_error())
    return status
