"""numpy/ctypes front end of the CPU oracle (oracle/liboracle_int8.so).

Test infrastructure: used by tests/ (and the smoke/bench checkers) to compute
expected values. Built by ``make -C oracle``.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# OMNI_ORACLE_LIBRARY may name the sanitised build (tests/sanitize_cpu.sh).
LIB = os.environ.get("OMNI_ORACLE_LIBRARY") or os.path.join(ROOT, "oracle", "liboracle_int8.so")

_P = ctypes.c_void_p
_I = ctypes.c_int64


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class Oracle:
    def __init__(self):
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB)
        sig = {
            "oracle_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "oracle_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "oracle_round_half_away": (ctypes.c_int32, [ctypes.c_float]),
            "oracle_unpack_i8": (None, [_P, _I, _P]),
            "oracle_pack_i8": (None, [_P, _I, _P]),
            "oracle_quantize_rows": (None, [_P, _I, _I, _I, _P, _P, _P]),
            "oracle_int8_acc": (None, [_P, _P, _I, _I, _I, _P]),
            "oracle_epilogue": (ctypes.c_float, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                                 ctypes.c_float, ctypes.c_float]),
            "oracle_int8_gemm": (None, [_P, _I, _I, _P, _P, _P, _I, _P]),
            "oracle_int8_gemm_threads": (None, [_P, _I, _I, _P, _P, _P, _I, _P, ctypes.c_int]),
            "oracle_w8a8_finish": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _P, _P]),
            "oracle_dequant_reference": (None, [_P, _I, _I, _P, _P, _P, _I, _P]),
            "oracle_w8a16_f64": (None, [_P, _I, _I, _P, _P, _P, _I, _P]),
            "oracle_w8a16_gemm": (None, [_P, _I, _I, _P, _P, _P, _I, _P]),
            "oracle_hadamard_sign_negative": (ctypes.c_int, [ctypes.c_uint64] * 3),
            "oracle_hadamard": (None, [_I, _P]),
            "oracle_rotate": (None, [_P, _I, _I, _I, _P]),
            "oracle_convrot_fwht": (None, [_P, _I, _I, _I, _P]),
            "oracle_convrot_quantize_fwht": (None, [_P, _I, _I, _I, _P, _P, _P]),
            "oracle_unpack_int4": (None, [_P, _I, _P]),
            "oracle_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "oracle_w4a16_dequant": (None, [_P, _P, _I, _I, _I, ctypes.c_int, _P]),
            "oracle_w4a16_f64": (None, [_P, _I, _I, _P, _P, _I, _P, _I, _P]),
            "oracle_w4a16_gemm": (None, [_P, _I, _I, _P, _P, _I, _P, _I, _P]),
            "oracle_f16_linear_f64": (None, [_P, _I, _I, _P, _I, _P]),
            "oracle_f16_gemv": (None, [_P, _I, _I, _P, _I, _P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        self.L = L

    # -- scalar helpers -------------------------------------------------
    def round_half_away(self, v):
        return self.L.oracle_round_half_away(float(v))

    def epilogue(self, acc, s, zero, rs, ws):
        return self.L.oracle_epilogue(acc, s, zero, rs, ws)

    # -- array helpers (numpy in, numpy out) ----------------------------
    def f16_to_f32(self, h):
        h = np.ascontiguousarray(h, dtype=np.uint16)
        return np.array([self.L.oracle_f16_to_f32(int(v)) for v in h.ravel()],
                        dtype=np.float32).reshape(h.shape)

    def f32_to_f16_bits(self, f):
        f = np.ascontiguousarray(f, dtype=np.float32)
        return np.array([self.L.oracle_f32_to_f16(float(v)) for v in f.ravel()],
                        dtype=np.uint16).reshape(f.shape)

    def unpack_i8(self, words):
        words = np.ascontiguousarray(words, dtype=np.int32)
        out = np.empty(words.size * 4, dtype=np.int8)
        self.L.oracle_unpack_i8(_p(words), words.size, _p(out))
        return out

    def pack_i8(self, codes):
        codes = np.ascontiguousarray(codes, dtype=np.int8).ravel()
        out = np.empty(codes.size // 4, dtype=np.int32)
        self.L.oracle_pack_i8(_p(codes), codes.size, _p(out))
        return out

    def quantize_rows(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, width = x.shape
        codes = np.empty((rows, width), dtype=np.int8)
        scale = np.empty(rows, dtype=np.float32)
        total = np.empty(rows, dtype=np.int32)
        self.L.oracle_quantize_rows(_p(x), rows, width, width, _p(codes), _p(scale), _p(total))
        return codes, scale, total

    def int8_acc(self, codes, w):
        codes = np.ascontiguousarray(codes, dtype=np.int8)
        w = np.ascontiguousarray(w, dtype=np.int8)
        rows, width = codes.shape
        columns = w.shape[0]
        acc = np.empty((rows, columns), dtype=np.int32)
        self.L.oracle_int8_acc(_p(codes), _p(w), rows, columns, width, _p(acc))
        return acc

    def int8_gemm(self, x, w, scale, zero):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.int8)
        scale = np.ascontiguousarray(scale, dtype=np.float32)
        zero = np.ascontiguousarray(zero, dtype=np.int32)
        rows, width = x.shape
        columns = w.shape[0]
        out = np.empty((rows, columns), dtype=np.float32)
        self.L.oracle_int8_gemm(_p(x), rows, width, _p(w), _p(scale), _p(zero), columns, _p(out))
        return out

    def int8_gemm_threads(self, x, w, scale, zero, threads):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.int8)
        scale = np.ascontiguousarray(scale, dtype=np.float32)
        zero = np.ascontiguousarray(zero, dtype=np.int32)
        rows, width = x.shape
        columns = w.shape[0]
        out = np.empty((rows, columns), dtype=np.float32)
        self.L.oracle_int8_gemm_threads(_p(x), rows, width, _p(w), _p(scale), _p(zero), columns,
                                        _p(out), int(threads))
        return out

    def w8a8_finish(self, acc, row_sum, row_scale, w_scale, w_zero, bias=None):
        acc = np.ascontiguousarray(acc, dtype=np.int32)
        rows, columns = acc.shape
        row_sum = np.ascontiguousarray(row_sum, dtype=np.int32)
        row_scale = np.ascontiguousarray(row_scale, dtype=np.float32)
        w_scale = np.ascontiguousarray(w_scale, dtype=np.float32)
        w_zero = np.ascontiguousarray(w_zero, dtype=np.int32)
        bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        o32 = np.empty((rows, columns), dtype=np.float32)
        o16 = np.empty((rows, columns), dtype=np.uint16)
        self.L.oracle_w8a8_finish(_p(acc), _p(row_sum), _p(row_scale), _p(w_scale), _p(w_zero),
                                  _p(bias), rows, columns, _p(o32), _p(o16))
        return o32, o16

    def dequant_reference(self, x, w, scale, zero):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.int8)
        scale = np.ascontiguousarray(scale, dtype=np.float32)
        zero = np.ascontiguousarray(zero, dtype=np.int32)
        rows, width = x.shape
        columns = w.shape[0]
        out = np.empty((rows, columns), dtype=np.float32)
        self.L.oracle_dequant_reference(_p(x), rows, width, _p(w), _p(scale), _p(zero), columns,
                                        _p(out))
        return out

    def w8a16_f64(self, x16, w, scale16, bias16=None):
        x16 = np.ascontiguousarray(x16).view(np.uint16)
        w = np.ascontiguousarray(w, dtype=np.int8)
        scale16 = np.ascontiguousarray(scale16).view(np.uint16)
        bias16 = None if bias16 is None else np.ascontiguousarray(bias16).view(np.uint16)
        rows, width = x16.shape
        columns = w.shape[0]
        out = np.empty((rows, columns), dtype=np.float64)
        self.L.oracle_w8a16_f64(_p(x16), rows, width, _p(w), _p(scale16), _p(bias16), columns,
                                _p(out))
        return out

    def w8a16_gemm(self, x16, w, scale16, bias16=None):
        x16 = np.ascontiguousarray(x16).view(np.uint16)
        w = np.ascontiguousarray(w, dtype=np.int8)
        scale16 = np.ascontiguousarray(scale16).view(np.uint16)
        bias16 = None if bias16 is None else np.ascontiguousarray(bias16).view(np.uint16)
        rows, width = x16.shape
        columns = w.shape[0]
        out = np.empty((rows, columns), dtype=np.uint16)
        self.L.oracle_w8a16_gemm(_p(x16), rows, width, _p(w), _p(scale16), _p(bias16), columns,
                                 _p(out))
        return out.view(np.float16)

    def hadamard(self, size):
        out = np.empty((size, size), dtype=np.float32)
        self.L.oracle_hadamard(size, _p(out))
        return out

    def rotate(self, x, group=256):
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, width = x.shape
        out = np.empty_like(x)
        self.L.oracle_rotate(_p(x), rows, width, group, _p(out))
        return out

    # -- W4A16 (crates/minicpm-v/src/quant.rs) --------------------------------
    def convrot_fwht(self, x):
        """u = 16 r of each group of 256, by the kernel's fast transform."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, width = x.shape
        u = np.empty((rows, width), dtype=np.float32)
        self.L.oracle_convrot_fwht(_p(x), rows, width, width, _p(u))
        return u

    def convrot_quantize_fwht(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, width = x.shape
        codes = np.empty((rows, width), dtype=np.int8)
        scale = np.empty(rows, dtype=np.float32)
        total = np.empty(rows, dtype=np.int32)
        self.L.oracle_convrot_quantize_fwht(_p(x), rows, width, width, _p(codes), _p(scale),
                                            _p(total))
        return codes, scale, total

    def unpack_int4(self, packed):
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        out = np.empty(packed.size * 2, dtype=np.int8)
        self.L.oracle_unpack_int4(_p(packed), packed.size, _p(out))
        return out

    def w4a16_dequant(self, packed, scale_bf16, rows, width, group=128, f16_round=False):
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        scale_bf16 = np.ascontiguousarray(scale_bf16).view(np.uint16)
        out = np.empty((rows, width), dtype=np.float32)
        self.L.oracle_w4a16_dequant(_p(packed), _p(scale_bf16), rows, width, group, int(f16_round),
                                    _p(out))
        return out

    def w4a16_f64(self, x16, packed, scale_bf16, group=128, bias16=None):
        x16 = np.ascontiguousarray(x16).view(np.uint16)
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        scale_bf16 = np.ascontiguousarray(scale_bf16).view(np.uint16)
        bias16 = None if bias16 is None else np.ascontiguousarray(bias16).view(np.uint16)
        rows, width = x16.shape
        columns = packed.shape[0]
        out = np.empty((rows, columns), dtype=np.float64)
        self.L.oracle_w4a16_f64(_p(x16), rows, width, _p(packed), _p(scale_bf16), group, _p(bias16),
                                columns, _p(out))
        return out

    def w4a16_gemm(self, x16, packed, scale_bf16, group=128, bias16=None):
        x16 = np.ascontiguousarray(x16).view(np.uint16)
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        scale_bf16 = np.ascontiguousarray(scale_bf16).view(np.uint16)
        bias16 = None if bias16 is None else np.ascontiguousarray(bias16).view(np.uint16)
        rows, width = x16.shape
        columns = packed.shape[0]
        out = np.empty((rows, columns), dtype=np.uint16)
        self.L.oracle_w4a16_gemm(_p(x16), rows, width, _p(packed), _p(scale_bf16), group, _p(bias16),
                                 columns, _p(out))
        return out.view(np.float16)

    def f16_linear_f64(self, x16, w16):
        """x f16 [rows, width], w f16 [columns, width] -> f64 [rows, columns]."""
        x16 = np.ascontiguousarray(x16).view(np.uint16)
        w16 = np.ascontiguousarray(w16).view(np.uint16)
        rows, width = x16.shape
        columns = w16.shape[0]
        out = np.empty((rows, columns), dtype=np.float64)
        self.L.oracle_f16_linear_f64(_p(x16), rows, width, _p(w16), columns, _p(out))
        return out

    def f16_gemv(self, x16, w16):
        """The reference GEMV's f32 lane-strided sums, cast to f16."""
        x16 = np.ascontiguousarray(x16).view(np.uint16)
        w16 = np.ascontiguousarray(w16).view(np.uint16)
        rows, width = x16.shape
        columns = w16.shape[0]
        out = np.empty((rows, columns), dtype=np.uint16)
        self.L.oracle_f16_gemv(_p(x16), rows, width, _p(w16), columns, _p(out))
        return out.view(np.float16)
