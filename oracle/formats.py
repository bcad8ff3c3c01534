"""Number-format codecs in numpy (oracle; test infrastructure only).

Pinned exhaustively against closed forms and torch's float8_e4m3fn / float16 /
bfloat16 dtypes (tests/test_oracle_formats.py).
"""
import numpy as np

F32 = np.float32


# ----------------------------------------------------------------- bf16
def bf16_bits(f):
    """fp32 -> bf16 bit patterns (uint16), round to nearest even; NaN stays a
    quiet NaN.  (torch's .to(torch.bfloat16), Triton's .to(tl.bfloat16))"""
    f = np.ascontiguousarray(f, dtype=F32)
    u = f.view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(f)
    r = np.where(nan, ((u >> 16) | 0x40), r)
    return (r & 0xFFFF).astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def round_bf16(f):
    """fp32 values rounded to bf16 precision, returned as fp32."""
    return bf16_to_f32(bf16_bits(f))


# ----------------------------------------------------------------- fp16
def f16_round(f):
    """fp32 -> fp16 (IEEE round to nearest even) -> fp32."""
    return np.asarray(f, dtype=F32).astype(np.float16).astype(F32)


# ----------------------------------------------------------------- e4m3fn
def _e4m3_table():
    v = np.zeros(256, dtype=np.float64)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 7
        if e == 15 and m == 7:
            v[b] = np.nan
        elif e == 0:
            v[b] = s * (m / 8.0) * 2.0 ** -6
        else:
            v[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return v.astype(F32)


E4M3 = _e4m3_table()                       # code -> value (OCP e4m3fn: bias 7, no inf)
_E4M3_POS = E4M3[:127].astype(np.float64)  # codes 0..126: 0 .. 448, increasing


def e4m3_decode(codes):
    return E4M3[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(v, saturate=False):
    """fp32 -> e4m3fn codes, round to nearest even.  Without `saturate`,
    |v| >= 480 becomes NaN (torch's float8_e4m3fn cast); with it, values clamp
    to +-448 first (OCP MX conversion)."""
    v = np.asarray(v, dtype=F32).astype(np.float64)
    a = np.abs(v)
    if saturate:
        a = np.minimum(a, 448.0)
    hi = np.searchsorted(_E4M3_POS, a, side="left")          # first table value >= a
    hi_c = np.minimum(hi, 126)
    lo_c = np.maximum(hi - 1, 0)
    hv = np.where(hi <= 126, _E4M3_POS[hi_c], 480.0)         # 480: first value past 448
    lv = _E4M3_POS[lo_c]
    exact = (hi <= 126) & (hv == a)
    dl, dh = a - lv, hv - a
    take_hi = (dh < dl) | ((dh == dl) & ((hi % 2) == 0))      # ties to even code
    code = np.where(exact, hi_c, np.where(take_hi, hi, lo_c))
    nan = np.isnan(v) | (code >= 127)
    sign = (np.signbit(v)).astype(np.int64) << 7
    out = np.where(nan, 0x7F, code) | np.where(nan, 0, sign)
    return out.astype(np.uint8)


def e4m3_round(v, saturate=False):
    return e4m3_decode(e4m3_encode(v, saturate))


# ----------------------------------------------------------------- e8m0
def e8m0_to_f32(e):
    """2^(e - 127) in fp32, as exp2((e - 127).float()) gives it (e = 255 -> inf)."""
    e = np.asarray(e, dtype=np.int64)
    return np.exp2((e - 127).astype(np.float64)).astype(F32)


# ----------------------------------------------------------------- e2m1
E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], dtype=F32)


def e2m1_decode(nib):
    return E2M1[np.asarray(nib, dtype=np.uint8) & 15]
