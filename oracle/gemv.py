"""Dequantize-then-matmul GEMV semantics (oracle; test infrastructure only).

y[m, n] = sum_k x[m, k] * bf16(deq(W)[n, k]), fp32 accumulation, cast to the
output dtype — the reference kernels' arithmetic (x/fp4x_kernels.py:9-176,
:304-325) with the summation order left to the accumulator (numpy's fp32
matmul here; oracle.ordered replays the HIP kernels' exact order).
"""
import numpy as np

from .formats import F32, round_bf16
from . import quant


def operand(fmt, *planes, **kw):
    """The bf16 weight operand (as fp32 values) each kernel feeds to its dot.
    fmt: mx8 (w, s) | w8 (q, s) | w6 (L, H, S) | nv4 (P, S_codes) |
    int2 (P, S[, scale_fmt])."""
    if fmt == "mx8":
        return round_bf16(quant.mx8_dequant(*planes))            # exact in bf16
    if fmt == "w8":
        return round_bf16(quant.dequant_w8(*planes))             # x/fp4x_kernels.py:129
    if fmt == "w6":
        return round_bf16(quant.dequant_w6(*planes))             # :170
    if fmt == "nv4":
        return round_bf16(quant.dequant_nv4_operand(*planes))    # :92 (exact in bf16)
    if fmt == "int2":
        return round_bf16(quant.dequant_int2(*planes, **kw))     # :321-322
    raise ValueError(fmt)


def matmul_f32(x, w_op):
    """fp32-accumulated x @ w_op.T for bf16-valued fp32 inputs."""
    return np.asarray(x, F32) @ np.asarray(w_op, F32).T


def cast(y, out_dtype):
    if out_dtype in ("bf16", "bfloat16"):
        return round_bf16(y)
    if out_dtype in ("f16", "float16"):
        return y.astype(np.float16).astype(F32)
    return np.asarray(y, F32)


def mx8_linear(x, w, s, out_dtype="bf16"):
    return cast(matmul_f32(x, operand("mx8", w, s)), out_dtype)


def w8_linear(x, q, s, out_dtype="bf16"):
    return cast(matmul_f32(x, operand("w8", q, s)), out_dtype)


def w6_linear(x, L, H, S, out_dtype="bf16"):
    return cast(matmul_f32(x, operand("w6", L, H, S)), out_dtype)


def nv4_linear(x, P, S_codes, gs, out_dtype="bf16"):
    """gs multiplies the accumulated sum (x/fp4x_kernels.py:94)."""
    return cast(matmul_f32(x, operand("nv4", P, S_codes)) * F32(gs), out_dtype)


def int2_logits(x, P, S, out_dtype="f32", scale_fmt="fp16", RS=None):
    y = matmul_f32(x, operand("int2", P, S, scale_fmt=scale_fmt))
    if RS is not None:
        y = y * np.asarray(RS, F32)[None, :]                     # x/fp4x_kernels.py:323-324
    return cast(y, out_dtype)


def within_tol(got, ref, rel=2e-3, abs_=1e-2):
    """|got - ref| <= abs_ + rel * |ref| elementwise (the GEMV parity bar)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.all(np.abs(got - ref) <= abs_ + rel * np.abs(ref))
