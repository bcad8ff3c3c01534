"""ctypes binding of libfp4x.so (the HIP kernels' C ABI, include/fp4x.h).

The library must be built (build.py); loading fails loudly otherwise.  torch
is imported first so the library binds to the HIP runtime torch already
loaded (both use the soname libamdhip64.so.7) and shares its streams.
"""
import ctypes
import os

import torch  # noqa: F401  (HIP runtime first)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfp4x.so")

OK, ERR_ARG, ERR_LAUNCH = 0, -1, -2
DT_BF16, DT_F32, DT_F16, DT_E4M3 = 0, 1, 2, 3
FMT_MX8, FMT_W8_F32, FMT_W8_F16, FMT_W6, FMT_NV4, FMT_INT2_F16, FMT_INT2_E4M3, FMT_BF16 = range(8)

_P, _I, _I64, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
_SIGS = {
    "fp4x_last_error": ([], ctypes.c_char_p),
    "fp4x_abi_version": ([], _I),
    "fp4x_layout": ([_I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)], _I),
    "fp4x_splitk_sizes": ([_I, _I, _I, _I, _I, _I, ctypes.POINTER(_I64), ctypes.POINTER(_I64)], _I),
    "fp4x_mx8_linear": ([_P, _I64, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P], _I),
    "fp4x_bf16_linear": ([_P, _I64, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P], _I),
    "fp4x_w8_linear": ([_P, _I64, _P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _P, _P], _I),
    "fp4x_w8_linear_layers": ([_P, _I64, _I64, _P, _I64, _P, _I, _I64, _P, _I, _I64, _I, _I, _I, _I, _I, _P, _P, _P],
                              _I),
    "fp4x_w6_linear": ([_P, _I64, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P], _I),
    "fp4x_nv4_linear": ([_P, _I64, _P, _P, _F, _P, _I, _I, _I, _I, _I, _P, _P, _P], _I),
    "fp4x_int2_logits": ([_P, _I64, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _P], _I),
    "fp4x_topk_rows": ([_P, _I, _I64, _I, _I, _I, _P, _P, _I64, _P], _I),
    "fp4x_topk_workspace_size": ([_I, _I], _I64),
    "fp4x_int2_topk": ([_P, _I64, _P, _P, _I, _P, _P, _I, _I64, _I, _I, _I, _I, _I, _P, _I, _P, _I64, _P], _I),
    "fp4x_int2_topk_noalloc": ([_P, _I64, _P, _P, _I, _P, _P, _I, _I64, _I, _I, _I, _I, _I, _P, _I, _P], _I),
    "fp4x_int2_topk_noalloc_limit": ([], _I64),
    "fp4x_refine_mx8": ([_P, _I, _I64, _P, _P, _I, _I, _P, _P, _I, _I, _P], _I),
    "fp4x_refine_nv4": ([_P, _P, _P, _I, _I, _P, _P, ctypes.c_float, _I, _I, _P], _I),
    "fp4x_scatter_draft": ([_P, _I64, _P, _P, _P, _I64, _P, _I, _I, _I64, _P], _I),
    "fp4x_draft_nv4": ([_P, _I64, _P, _P, _P, _I64, _P, _P, ctypes.c_float, _P, _I, _I, _I, _I64, _P], _I),
    "fp4x_quantize": ([_I, _P, _P, ctypes.c_float, _I64, _I, _I, _I, _I, ctypes.c_float, _P, _P, _P, _P], _I),
    "fp4x_quantize_w6_clip": ([_I, _P, _P, ctypes.c_float, _I64, _I, _I, _I, _P, _P, _P, _P], _I),
    "fp4x_absmax": ([_I, _P, _P, ctypes.c_float, _I64, _I, _P, _P], _I),
    "fp4x_hc_down": ([_P, _I64, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P], _I),
    "fp4x_hc_up": ([_P, _I64, _P, _P, _I, _P, _I64, _P, _I, _I, _I, _I, _I, _P], _I),
    "fp4x_hc_mix": ([_P, _I64, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _P, _I64, _P, _I, _I,
                     _P], _I),
    "fp4x_hc_scaled_silu": ([_P, _I64, _P, _I, _I, _I, _P], _I),
    "fp4x_hc_gate_mean": ([_P, _I64, _P, _I64, _P, _I, _I, _I, _P], _I),
    "fp4x_dequant_bf16": ([_I, _P, _P, _P, _I, _I, _I, _P, _P], _I),
    "fp4x_mx8_dequant": ([_P, _P, _I, _I, _P, _P], _I),
    "fp4x_reload_env": ([], _I),
    "fp4x_read_ceiling": ([_P, _I64, _I, _I, _P, _P], _I),
    "fp4x_hold_cus": ([_I, _I64, _I, _P, _P], _I),
}
ABI_VERSION = 12

_LIB = None


def lib():
    """The loaded library (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"fp4x: {LIB_PATH} is not built; run build.py (hipcc, gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        if L.fp4x_abi_version() != ABI_VERSION:
            raise RuntimeError("fp4x: libfp4x.so ABI version mismatch; rebuild")
        _LIB = L
    return _LIB


def check(rc, what):
    if rc != OK:
        msg = lib().fp4x_last_error().decode(errors="replace")
        if rc == ERR_ARG:
            raise ValueError(f"fp4x {what}: {msg}")
        raise RuntimeError(f"fp4x {what}: {msg}")


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def layout(fmt, k_slice):
    lpr, cpl = ctypes.c_int(), ctypes.c_int()
    check(lib().fp4x_layout(fmt, k_slice, ctypes.byref(lpr), ctypes.byref(cpl)), "layout")
    return lpr.value, cpl.value


def splitk_sizes(fmt, M, N, K, ksplit, batch=1):
    pf, nt = ctypes.c_int64(), ctypes.c_int64()
    check(lib().fp4x_splitk_sizes(fmt, M, N, K, ksplit, batch, ctypes.byref(pf), ctypes.byref(nt)), "splitk_sizes")
    return pf.value, nt.value


def reload_env():
    """Re-read the library's FP4X_* path switches (read once otherwise)."""
    check(lib().fp4x_reload_env(), "reload_env")


DTYPE_CODE = {torch.bfloat16: DT_BF16, torch.float32: DT_F32, torch.float16: DT_F16}
