"""ctypes front end of ordered.c, the rescore kernels' exact fma order, plus
the float64 sums and error bounds the MFMA-accumulated GEMVs are checked
against (oracle; test infrastructure only)."""
import ctypes
import os

import numpy as np

from . import build as _build

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        src = os.path.join(os.path.dirname(_build.SO), "..", "ordered.c")
        if not os.path.exists(_build.SO) or os.path.getmtime(_build.SO) < os.path.getmtime(src):
            _build.build()
        L = ctypes.CDLL(_build.SO)
        P = ctypes.c_void_p
        L.oracle_ordered_gemv.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_float, P]
        L.oracle_int2_operand.argtypes = [P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, P]
        _LIB = L
    return _LIB


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def ordered_gemv(x_bits, w_bits, kpc, lpr, ksplit=1, gs=1.0, rows=None):
    """fp32 sums in the rescore kernels' order (ordered.c): per lane a chain of
    IEEE fma over its chunks, a butterfly over the lpr lanes, slices times gs
    added in order.  x_bits uint16 bf16 [M, K]; w_bits uint16 bf16 operand
    [R, K]; rows (int64 [M, N]) gathers weight rows per output, else N = R.
    Returns float32 [M, N]."""
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
                              float(gs), _p(out))
    return out


def step_bound(x, w, kpc, lpr, ksplit=1):
    """|error| bound of an fma-ordered sum against the exact one: every fma and
    butterfly addition rounds once (at most half an ulp of a partial that is
    itself at most sum_k |x_k w_k|), so the error is at most
    n_steps * 2^-24 * sum_k |x_k w_k|; taken here with 2^-23 per step.
    x, w: fp32 values [M, K], [N, K]."""
    K = x.shape[1]
    chunks = K // ksplit // kpc
    cpl = -(-chunks // lpr)
    n_steps = cpl * kpc + max(lpr.bit_length() - 1, 0) + ksplit + 1
    l1 = np.abs(np.asarray(x, np.float64)) @ np.abs(np.asarray(w, np.float64)).T
    return n_steps * 2.0 ** -23 * l1


def mfma_bound(x, w, ksplit=1):
    """|error| bound of an MFMA-accumulated sum against the exact sum:
    v_mfma_f32_16x16x32_bf16 adds 32 products to its accumulator with an
    error of at most 2.53 * 2^-23 * (L1 of those terms) (measured on random
    operands spanning 2^48), chained over K/32 instructions, plus the wave and
    K-slice additions.  x, w: fp32 values [M, K], [N, K]."""
    K = x.shape[1]
    n_events = 3 * (K // 32) + 16 + ksplit
    l1 = np.abs(np.asarray(x, np.float64)) @ np.abs(np.asarray(w, np.float64)).T
    return n_events * 2.0 ** -23 * l1


def exact_sum(x, w):
    """float64 x @ w.T: for bf16-valued operands every product is exact in
    float64, and the float64 summation error at these sizes lies far below
    the fp32 bounds it is compared with."""
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T


def int2_operand_bits(P, S_f16, G):
    """bf16 operand bits of an INT2 fp16-scale head, [N, K]."""
    P = np.ascontiguousarray(P, np.uint8)
    S = np.ascontiguousarray(np.asarray(S_f16, np.float16).view(np.uint16))
    N = P.shape[0]
    K = P.shape[1] * 4
    out = np.empty((N, K), np.uint16)
    lib().oracle_int2_operand(_p(P), _p(S), N, K, G, _p(out))
    return out
