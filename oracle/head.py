"""Fast target LM head flow (oracle; test infrastructure only).

x/fp4patch.py:370-378: coarse = int2_logits(h, P, S, V, out_dtype=bf16);
idx = topk(coarse, C); refine_mx8_(coarse, h, idx, w, s) overwrites the C
selected logits with exact MXFP8 dot products.  The top-C selection uses the
total order (value descending, index ascending), -0 equal to +0 and NaN
largest; the sums replay the kernels' order through oracle.ordered so that
coarse values, the selected set and the refined logits are exact.
"""
import numpy as np

from .formats import F32, bf16_bits, bf16_to_f32
from . import ordered, quant


def order_keys(bits):
    """bf16 bits -> uint32 keys increasing with the value."""
    b = np.asarray(bits, np.uint16).astype(np.uint32)
    b = np.where((b & 0x7FFF) == 0, 0, b)
    nan = ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)
    b = np.where(nan, 0x7FC0, b)
    return np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000).astype(np.uint32)


def topk_total_order(bits, C):
    """Indices [M, C] of the C largest bf16 values per row, sorted by
    (value desc, index asc)."""
    keys = order_keys(bits).astype(np.int64)
    M, V = keys.shape
    comp = (keys << 32) | (0xFFFFFFFF - np.arange(V, dtype=np.int64))[None, :]
    part = np.argpartition(-comp, C - 1, axis=1)[:, :C]
    sel = np.take_along_axis(comp, part, 1)
    order = np.argsort(-sel, axis=1, kind="stable")
    return np.take_along_axis(part, order, 1).astype(np.int64)


def int2_coarse(x_bits, P, S, G, lpr):
    """Exact coarse sums (fp32, kernel order) of the fp16-scale INT2 head."""
    w = ordered.int2_operand_bits(P, S, G)
    return ordered.ordered_gemv(x_bits, w, kpc=64, lpr=lpr)


def mx8_rows(x_bits, w_codes, s_u8, rows, lpr):
    """Exact MXFP8 sums of the gathered rows rows [M, C]: the rescore kernel's
    order with IEEE fma steps (ordered model 2)."""
    uniq, inv = np.unique(rows, return_inverse=True)
    w_op = bf16_bits(quant.mx8_dequant(w_codes[uniq], s_u8[uniq]))
    return ordered.ordered_gemv(x_bits, w_op, kpc=16, lpr=lpr, rows=inv.reshape(rows.shape), mode=ordered.FMA)


def fast_head(x_bits, P, S, G, w_codes, s_u8, C, lpr_int2, lpr_mx8):
    """Returns (coarse bf16 bits [M, V], idx [M, C], logits bf16 bits [M, V])."""
    coarse = bf16_bits(int2_coarse(x_bits, P, S, G, lpr_int2))
    idx = topk_total_order(coarse, C)
    exact = bf16_bits(mx8_rows(x_bits, w_codes, s_u8, idx, lpr_mx8))
    out = coarse.copy()
    np.put_along_axis(out, idx, exact, 1)
    return coarse, idx, out


def full_mx8_logits(x_bits, w_codes, s_u8):
    """Exact-weight full-vocabulary logits (fp32, numpy order) for argmax
    agreement checks."""
    return bf16_to_f32(x_bits).astype(F32) @ quant.mx8_dequant(w_codes, s_u8).T


# ----------------------------------------------------------------- draft head
def nv4_rows(x_bits, P, S_codes, gs, rows, lpr):
    """Exact NVFP4 logits [M, C] of the gathered rows rows [M, C], times gs:
    the rescore kernel's order with IEEE fma steps (ordered model 2); the
    operand e2m1 * e4m3 is exact in bf16.  [x/fp4x_kernels.py:391-415]"""
    uniq, inv = np.unique(rows, return_inverse=True)
    w_op = bf16_bits(quant.dequant_nv4_operand(P[uniq], S_codes[uniq]))
    return ordered.ordered_gemv(x_bits, w_op, kpc=32, lpr=lpr, gs=gs, rows=inv.reshape(rows.shape),
                                mode=ordered.FMA)


def draft_head(x_bits, P2, S2, G, P, S_codes, gs, ids, vocab, dc, lpr_int2, lpr_nv4):
    """The draft head over a token subset ids (x/fp4patch.py:312-320): INT2
    coarse over the subset rows, the top dc by the total order, their exact
    NVFP4 logits, scattered into a -inf bf16 row of the full vocabulary.
    Returns (cand [M, dc] subset positions, vals fp32 [M, dc], full bf16 bits)."""
    coarse = bf16_bits(int2_coarse(x_bits, P2, S2, G, lpr_int2))
    cand = topk_total_order(coarse, dc)
    vals = nv4_rows(x_bits, P, S_codes, gs, cand, lpr_nv4)
    full = np.full((x_bits.shape[0], vocab), 0xFF80, np.uint16)          # bf16 -inf
    np.put_along_axis(full, np.asarray(ids, np.int64)[cand], bf16_bits(vals), 1)
    return cand, vals, full
