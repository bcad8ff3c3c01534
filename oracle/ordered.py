"""ctypes front end of ordered.c: the HIP kernels' exact summation order
(oracle; test infrastructure only)."""
import ctypes
import os

import numpy as np

from . import build as _build

# v_dot2_f32_bf16 rounding model; tests/test_gpu_dot2.py checks it against
# the hardware on crafted and random operands (see ordered.c for the models).
DOT2_MODE = 0

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(_build.SO):
            _build.build()
        L = ctypes.CDLL(_build.SO)
        P = ctypes.c_void_p
        L.oracle_dot2_batch.argtypes = [P, P, P, P, ctypes.c_int64, ctypes.c_int]
        L.oracle_ordered_gemv.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, P]
        L.oracle_int2_operand.argtypes = [P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, P]
        _LIB = L
    return _LIB


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def dot2(a, b, c, mode=None):
    """Elementwise dot2 model: a, b uint32 bf16 pairs, c float32."""
    a = np.ascontiguousarray(a, np.uint32)
    b = np.ascontiguousarray(b, np.uint32)
    c = np.ascontiguousarray(c, np.float32)
    out = np.empty(a.shape, np.float32)
    lib().oracle_dot2_batch(_p(a), _p(b), _p(c), _p(out), a.size, DOT2_MODE if mode is None else mode)
    return out


def ordered_gemv(x_bits, w_bits, kpc, lpr, ksplit=1, gs=1.0, rows=None, mode=None):
    """fp32 sums in kernel order.  x_bits uint16 bf16 [M, K]; w_bits uint16
    bf16 operand [R, K]; rows (int64 [M, N]) gathers weight rows per output,
    else N = R.  Returns float32 [M, N]."""
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    w_bits = np.ascontiguousarray(w_bits, np.uint16)
    M, K = x_bits.shape
    if rows is not None:
        rows = np.ascontiguousarray(rows, np.int64)
        N = rows.shape[1]
    else:
        N = w_bits.shape[0]
    out = np.empty((M, N), np.float32)
    lib().oracle_ordered_gemv(_p(x_bits), _p(w_bits), None if rows is None else _p(rows), M, N, K, kpc, ksplit, lpr,
                              float(gs), DOT2_MODE if mode is None else mode, _p(out))
    return out


def int2_operand_bits(P, S_f16, G):
    """bf16 operand bits of an INT2 fp16-scale head, [N, K]."""
    P = np.ascontiguousarray(P, np.uint8)
    S = np.ascontiguousarray(np.asarray(S_f16, np.float16).view(np.uint16))
    N = P.shape[0]
    K = P.shape[1] * 4
    out = np.empty((N, K), np.uint16)
    lib().oracle_int2_operand(_p(P), _p(S), N, K, G, _p(out))
    return out
