"""Fast target LM head and draft head flows (oracle; test infrastructure only).

Target head, x/fp4patch.py:370-378: coarse = int2_logits(h, P, S, V,
out_dtype=bf16); idx = torch.topk(coarse, C); refine_mx8_(coarse, h, idx, w, s)
overwrites the C selected logits with exact MXFP8 dot products.

Draft head, x/fp4patch.py:312-320: co = int2_logits(h, *coarse, n) in fp32
(int2_logits' default out_dtype); cand = torch.topk(co, dc); vals =
refine_nv4(h, cand, ...); a -inf bf16 row of the full vocabulary receives
bf16(vals) (times 1/t) at ids[cand].

Restated semantics:
  - coarse sums: the reference accumulates in fp32 in an order Triton leaves
    open; the oracle takes the exact sum (float64, exact products) rounded
    once to fp32, then to the output dtype.  An fp32 accumulator in any order
    lies within an error bound of it (oracle.ordered.mfma_bound for the HIP
    kernels' MFMA accumulation).
  - top-C: torch.topk's set under the total order value descending, then
    index ascending, with -0 equal to +0 and NaN largest (torch leaves the
    order among ties open; the HIP select fixes it this way).
  - rescore sums: exact products, fp32 fma in the HIP rescore kernels' order
    (oracle.ordered), which every fp32 accumulation order approximates within
    oracle.ordered.step_bound.
"""
import numpy as np

from .formats import F32, bf16_bits, bf16_to_f32
from . import ordered, quant


def order_keys(vals):
    """Order keys increasing with the value: bf16 bits (uint16) give uint32
    keys below 2^16, fp32 values (float32) keys below 2^32.  -0 maps to +0's
    key, every NaN to one key above +inf."""
    a = np.asarray(vals)
    if a.dtype == np.uint16:
        b = a.astype(np.uint32) << 16
    elif a.dtype == np.float32:
        b = np.ascontiguousarray(a).view(np.uint32).astype(np.uint32)
    else:
        raise TypeError(f"order_keys takes bf16 bits (uint16) or float32, got {a.dtype}")
    b = np.where((b & 0x7FFFFFFF) == 0, 0, b).astype(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    b = np.where(nan, 0x7FC00000, b).astype(np.uint32)
    key = np.where(b & 0x80000000, (~b) & 0xFFFFFFFF, b | 0x80000000).astype(np.uint32)
    return key >> 16 if a.dtype == np.uint16 else key


def topk_total_order(vals, C):
    """Indices [M, C] of the C largest values per row (bf16 bits uint16, or
    float32), sorted by (value desc, index asc)."""
    keys = order_keys(vals).astype(np.uint64)
    M, V = keys.shape
    comp = (keys << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - np.arange(V, dtype=np.uint64))[None, :]
    inv = ~comp                                   # ascending inv = descending comp (all distinct)
    part = np.argpartition(inv, C - 1, axis=1)[:, :C]
    sel = np.take_along_axis(inv, part, 1)
    order = np.argsort(sel, axis=1, kind="stable")
    return np.take_along_axis(part, order, 1).astype(np.int64)


def int2_coarse(x_bits, P, S, G, rows_per_chunk=16384):
    """Coarse INT2 logits (fp16 scales) as fp32: the exact sum of x . bf16
    operand rounded once to fp32.  x_bits uint16 [M, K]; P [V, K/4]; S fp16
    [V, K/G]."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    V = P.shape[0]
    out = np.empty((x.shape[0], V), F32)
    for r0 in range(0, V, rows_per_chunk):
        r1 = min(V, r0 + rows_per_chunk)
        w = bf16_to_f32(ordered.int2_operand_bits(P[r0:r1], S[r0:r1], G))
        out[:, r0:r1] = (x @ w.T.astype(np.float64)).astype(F32)
    return out


def mx8_rows(x_bits, w_codes, s_u8, rows, lpr):
    """Exact MXFP8 sums of the gathered rows rows [M, C]: the rescore kernel's
    fma order (oracle.ordered)."""
    uniq, inv = np.unique(rows, return_inverse=True)
    w_op = bf16_bits(quant.mx8_dequant(w_codes[uniq], s_u8[uniq]))
    return ordered.ordered_gemv(x_bits, w_op, kpc=16, lpr=lpr, rows=inv.reshape(rows.shape))


def fast_head(x_bits, P, S, G, w_codes, s_u8, C, lpr_mx8):
    """Returns (coarse bf16 bits [M, V], idx [M, C], logits bf16 bits [M, V])."""
    coarse = bf16_bits(int2_coarse(x_bits, P, S, G))
    idx = topk_total_order(coarse, C)
    exact = bf16_bits(mx8_rows(x_bits, w_codes, s_u8, idx, lpr_mx8))
    out = coarse.copy()
    np.put_along_axis(out, idx, exact, 1)
    return coarse, idx, out


def fast_head_argmax(x_bits, P, S, G, w_codes, s_u8, C, lpr_mx8, block=96):
    """Per row, the argmax (first index of the largest value) of fast_head's
    output, for many rows: the coarse pass runs over the head once for all
    rows, the top-C and the rescore per block of rows, so 1,000 rows of a
    248,320-row head stay within a few GB."""
    coarse = bf16_bits(int2_coarse(x_bits, P, S, G))
    am = np.empty(coarse.shape[0], np.int64)
    for b0 in range(0, coarse.shape[0], block):
        cb = coarse[b0:b0 + block]
        idx = topk_total_order(cb, C)
        out = cb.copy()
        np.put_along_axis(out, idx, bf16_bits(mx8_rows(x_bits[b0:b0 + block], w_codes, s_u8, idx, lpr_mx8)), 1)
        am[b0:b0 + block] = np.argmax(bf16_to_f32(out), -1)
    return am


def full_mx8_logits(x_bits, w_codes, s_u8):
    """Exact-weight full-vocabulary logits (fp32, numpy order) for argmax
    agreement checks."""
    return bf16_to_f32(x_bits).astype(F32) @ quant.mx8_dequant(w_codes, s_u8).T


# ----------------------------------------------------------------- draft head
def nv4_rows(x_bits, P, S_codes, gs, rows, lpr):
    """Exact NVFP4 logits [M, C] of the gathered rows rows [M, C], times gs:
    the rescore kernel's fma order (oracle.ordered); the operand e2m1 * e4m3
    is exact in bf16.  [x/fp4x_kernels.py:391-415]"""
    uniq, inv = np.unique(rows, return_inverse=True)
    w_op = bf16_bits(quant.dequant_nv4_operand(P[uniq], S_codes[uniq]))
    return ordered.ordered_gemv(x_bits, w_op, kpc=32, lpr=lpr, gs=gs, rows=inv.reshape(rows.shape))


def draft_head(x_bits, P2, S2, G, P, S_codes, gs, ids, vocab, dc, lpr_nv4, inv_t=None):
    """The draft head over a token subset ids (x/fp4patch.py:312-320): fp32
    INT2 coarse logits over the subset rows, the top dc of them by the total
    order, their exact NVFP4 logits (times inv_t in fp32 when given),
    scattered as bf16 into a -inf row of the full vocabulary.
    Returns (cand [M, dc] subset positions, vals fp32 [M, dc], full bf16 bits)."""
    coarse = int2_coarse(x_bits, P2, S2, G)
    cand = topk_total_order(coarse, dc)
    vals = nv4_rows(x_bits, P, S_codes, gs, cand, lpr_nv4)
    if inv_t is not None:
        vals = (vals * F32(inv_t)).astype(F32)
    full = np.full((x_bits.shape[0], vocab), 0xFF80, np.uint16)          # bf16 -inf
    np.put_along_axis(full, np.asarray(ids, np.int64)[cand], bf16_bits(vals), 1)
    return cand, vals, full
