"""Quantizers and dequantizers of the plugin's packed formats, restated in
numpy (oracle; test infrastructure only).

Each function follows the cited reference function step by step at its
floating-point rounding points: torch divides an fp32 tensor by a Python
scalar as an IEEE fp32 division by fp32(scalar), torch.round is round half to
even, torch.bucketize(right=False) sends ties to the lower bucket, and fp16 /
e4m3 casts round to nearest even.
"""
import numpy as np

from .formats import F32, E2M1, e4m3_encode, e4m3_decode, e8m0_to_f32, f16_round

ORDER = (0, 2, 1, 3)  # INT2: element j of each 4-group lives in bit pair ORDER[j]


def _groups(w, g):
    w = np.asarray(w, dtype=F32)
    n, k = w.shape
    return w.reshape(n, k // g, g)


# ----------------------------------------------------------------- W8 g64
def quantize_w8(w):
    """(q int8 [N,K], s fp32 [N,K/64]).  [x/fp4x_kernels.py:138-144]"""
    f = _groups(w, 64)
    s = np.maximum(np.abs(f).max(-1), F32(1e-12)) / F32(127.0)
    q = np.clip(np.rint(f / s[..., None]), -127, 127).astype(np.int8)
    return q.reshape(w.shape), s.astype(F32)


def dequant_w8(q, s):
    n, k = q.shape
    return (q.astype(F32).reshape(n, k // 64, 64) * np.asarray(s, F32)[..., None]).reshape(n, k)


# ----------------------------------------------------------------- W6 g32
def _w6_scale(f, qmax):
    return np.maximum(f16_round(np.abs(f).max(-1, keepdims=True) / F32(qmax)), F32(6.2e-5))


def quantize_w6(w, qmax=31, clip_search=0):
    """(L u8 [N,K/2], H u8 [N,K/4], S fp16 [N,K/32]).  [x/fp4x_kernels.py:179-202]
    clip_search > 0 picks, per group, the first scale with the strictly
    smallest squared error over the reference's clip grid: the factors of
    torch.linspace(0.70, 0.98, n) in fp32 (clip_grid), each error summed in
    fp32 in the order of torch's CPU sum over a 32-element row (sum_sq32)."""
    w = np.asarray(w, dtype=F32)
    n, k = w.shape
    f = _groups(w, 32)
    s = _w6_scale(f, qmax)
    if clip_search:
        def err(sc):
            d = np.clip(np.rint(f / sc), -qmax - 1, qmax) * sc - f
            return sum_sq32(d)
        best, bs = err(s), s
        for c in clip_grid(clip_search):
            sc = np.maximum(f16_round(s * c), F32(6.2e-5))
            e = err(sc)
            m = e < best
            best = np.where(m, e, best)
            bs = np.where(m, sc, bs)
        s = bs
    q = (np.clip(np.rint(f / s), -qmax - 1, qmax).astype(np.int32) + 32).reshape(n, k)
    lo, hi = q & 15, q >> 4
    L = (lo[:, 0::2] | (lo[:, 1::2] << 4)).astype(np.uint8)
    H = (hi[:, 0::4] | (hi[:, 2::4] << 2) | (hi[:, 1::4] << 4) | (hi[:, 3::4] << 6)).astype(np.uint8)
    S = s[..., 0].astype(np.float16)
    return L, H, S


def clip_grid(n):
    """torch.linspace(0.70, 0.98, n) as fp32 values: step = fp32((0.98 - 0.70)
    / (n - 1)) from the fp32 ends, then c_i = start + step * i below n // 2
    and end - step * (n - 1 - i) from there, each rounded once (a fused
    multiply-add; the float64 expression below is exact before its rounding)."""
    s, e = F32(0.70), F32(0.98)
    if n == 1:
        return [s]
    st = F32((e - s) / F32(n - 1))
    return [F32(float(s) + float(st) * i) if i < n // 2 else F32(float(e) - float(st) * (n - 1 - i))
            for i in range(n)]


def sum_sq32(d):
    """fp32 sum of the squares of the last axis (32 values) in the order of
    torch's CPU sum over a 32-element row: lane j adds elements j, j + 8,
    j + 16, j + 24 in turn, then lanes 0..7 are added in turn; keeps the axis."""
    d2 = (d * d).astype(F32)
    lane = [d2[..., j] for j in range(8)]
    for i in range(8, 32, 8):
        lane = [(lane[j] + d2[..., i + j]).astype(F32) for j in range(8)]
    acc = lane[0]
    for j in range(1, 8):
        acc = (acc + lane[j]).astype(F32)
    return acc[..., None]


def w6_codes(L, H):
    """6-bit codes c = lo | hi << 4 in [0, 63], [N, K]."""
    L = np.asarray(L, dtype=np.uint8)
    H = np.asarray(H, dtype=np.uint8)
    n = L.shape[0]
    k = L.shape[1] * 2
    lo = np.empty((n, k), dtype=np.int32)
    lo[:, 0::2] = L & 15
    lo[:, 1::2] = L >> 4
    hi = np.empty((n, k), dtype=np.int32)
    hi[:, 0::4] = H & 3
    hi[:, 2::4] = (H >> 2) & 3
    hi[:, 1::4] = (H >> 4) & 3
    hi[:, 3::4] = (H >> 6) & 3
    return lo | (hi << 4)


def dequant_w6(L, H, S):
    """fp32 (c - 32) * s.  [x/fp4x_kernels.py:161-170]"""
    q = (w6_codes(L, H) - 32).astype(F32)
    n, k = q.shape
    return (q.reshape(n, k // 32, 32) * np.asarray(S).astype(F32)[..., None]).reshape(n, k)


# ----------------------------------------------------------------- NVFP4
_MIDS = ((E2M1[1:8] + E2M1[0:7]) / F32(2)).astype(F32)


def quantize_nv4(w, rows=2048):
    """(P u8 [N,K/2], S e4m3 codes u8 [N,K/16], gs python float).
    [x/fp4x_kernels.py:277-300]"""
    w = np.asarray(w, dtype=F32)
    n, k = w.shape
    amax_all = 0.0
    for a in range(0, n, rows):
        amax_all = max(amax_all, float(np.abs(w[a:a + rows]).max()))
    gs = max(amax_all / 6.0 / 448.0, 1e-30)
    gs32 = F32(gs)
    f = _groups(w, 16)
    sc = np.clip(np.abs(f).max(-1, keepdims=True) / F32(6.0) / gs32, F32(2.0 ** -9), F32(448.0))
    sc_code = e4m3_encode(sc)
    sf = (e4m3_decode(sc_code) * gs32).astype(F32)     # fp32 product (the reference's sc.float() * gs)
    v = np.clip(f / sf, F32(-6), F32(6))               # fp32 division
    mag = np.searchsorted(_MIDS, np.abs(v), side="left").astype(np.int64)
    q = (mag | ((v < 0).astype(np.int64) << 3)).reshape(n, k)
    P = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return P, sc_code.reshape(n, k // 16), gs


def nv4_values(P):
    P = np.asarray(P, dtype=np.uint8)
    n = P.shape[0]
    v = np.empty((n, P.shape[1] * 2), dtype=F32)
    v[:, 0::2] = E2M1[P & 15]
    v[:, 1::2] = E2M1[P >> 4]
    return v


def dequant_nv4_operand(P, S_codes):
    """e2m1 * e4m3 per element (the bf16-exact dot operand, before gs).
    [x/fp4x_kernels.py:85-92]"""
    v = nv4_values(P)
    n, k = v.shape
    return (v.reshape(n, k // 16, 16) * e4m3_decode(S_codes)[..., None]).reshape(n, k)


def dequant_nv4(P, S_codes, gs):
    """fp32 (v * S) * gs: the exact product v * S, one fp32 rounding by gs.
    [x/fp4x_kernels.py:420-426]"""
    return (dequant_nv4_operand(P, S_codes) * F32(gs)).astype(F32)


# ----------------------------------------------------------------- INT2
def quantize_int2(w, scale_fmt="fp16", group=16):
    """fp16: (P u8 [N,K/4], S fp16 [N,K/G]); e4m3: (P, S e4m3 codes, rows fp32 [N]).
    [x/fp4x_kernels.py:330-351]"""
    w = np.asarray(w, dtype=F32)
    n, k = w.shape
    f = _groups(w, group)
    s = np.maximum(np.abs(f).max(-1, keepdims=True), F32(1e-8)) / F32(1.5)
    if scale_fmt == "fp16":
        S = s.astype(np.float16)
        sf = S.astype(F32)
        rows = None
    else:
        rs = s.max(1, keepdims=True) / F32(448.0)
        S = e4m3_encode(s / rs)
        sf = (e4m3_decode(S) * rs).astype(F32)         # fp32 product (s.float() * rs)
        rows = rs.reshape(n).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        idx = np.clip(np.floor(f / sf) + 2, 0, 3).astype(np.uint8).reshape(n, k // 4, 4)
    P = np.zeros((n, k // 4), dtype=np.uint8)
    for j in range(4):
        P |= (idx[..., j] << (2 * ORDER[j])).astype(np.uint8)
    S = S[..., 0]
    return (P, S) if scale_fmt == "fp16" else (P, S, rows)


def int2_codes(P):
    P = np.asarray(P, dtype=np.uint8)
    n = P.shape[0]
    return np.stack([(P >> (2 * ORDER[j])) & 3 for j in range(4)], -1).reshape(n, P.shape[1] * 4)


def dequant_int2(P, S, scale_fmt="fp16"):
    """fp32 (code - 1.5) * s per group.  [x/fp4x_kernels.py:353-357]"""
    c = int2_codes(P).astype(F32) - F32(1.5)
    n, k = c.shape
    sf = np.asarray(S).astype(F32) if scale_fmt == "fp16" else e4m3_decode(S)
    g = k // sf.shape[1]
    return (c.reshape(n, k // g, g) * sf[..., None]).reshape(n, k)


# ----------------------------------------------------------------- MXFP8
def mx8_dequant(w_codes, s_u8):
    """fp32 e4m3(w) * 2^(s - 127).  [x/fp4x_kernels.py:261-267]"""
    w = e4m3_decode(w_codes)
    n, k = w.shape
    return (w.reshape(n, k // 32, 32) * e8m0_to_f32(s_u8)[..., None]).reshape(n, k).astype(F32)   # exact in fp32


def quantize_mx8(w):
    """OCP Microscaling v1.0 MXFP8 (e4m3 elements, e8m0 shared scale per 32):
    shared exponent floor(log2(amax)) - 8 (8 = emax of e4m3), clamped to
    [-127, 127] (amax = 0 -> -127); elements w / 2^X rounded to nearest even
    with saturation at +-448.  Returns (w codes u8 [N,K], s u8 [N,K/32])."""
    f = _groups(w, 32)
    amax = np.abs(f).max(-1)
    bits = amax.view(np.uint32)
    e_amax = ((bits >> 23) & 0xFF).astype(np.int64) - 127   # floor(log2) for normals
    sub = (bits >> 23) == 0                                   # zero / fp32 subnormal
    e_amax = np.where(sub, -127 - 8, e_amax)                  # -> shared exponent -127 after clamp
    X = np.clip(e_amax - 8, -127, 127)
    scale = np.exp2(X.astype(np.float64))
    q = e4m3_encode((f.astype(np.float64) / scale[..., None]).astype(F32), saturate=True)
    n, k = np.asarray(w).shape
    return q.reshape(n, k), (X + 127).astype(np.uint8)


# ----------------------------------------------------------------- mixer prep
def interleave_up_rows(n, hc, bj):
    """Row order of HCFused.interleave_up: stored row j_tile*hc*bj + s*bj + t
    holds original row s*H + j_tile*bj + t.  [x/fp4x_kernels.py:512-517]"""
    h = n // hc
    return np.arange(n).reshape(hc, h // bj, bj).transpose(1, 0, 2).reshape(-1)
