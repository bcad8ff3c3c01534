"""Hyper-connection mixer semantics (oracle; test infrastructure only).

Rounding points of the fused mixer kernels (x/fp4x_kernels.py:460-464 and
:486-493), which follow b12x's scaled-SiLU and gate-mean ops:
  down:  di = bf16(sum); sc = bf16(di / hc); bot = bf16(sc * sigmoid(sc))
  up:    g = bf16(sum); gate = bf16(sigmoid(g)); term_s = bf16(nrm_s * gate_s);
         out = bf16((term_0 + term_1 + ... ) / hc), terms added in stream order
sigmoid is evaluated in float64 and rounded to fp32: the correctly rounded
fp32 sigmoid (checked against a 200-bit evaluation over bf16 sweeps).  The
reference's tl.sigmoid may round differently in the last fp32 bit: parity with
it is unpinned.
"""
import numpy as np

from .formats import F32, round_bf16
from . import gemv, quant


def sigmoid32(x):
    x = np.asarray(x, np.float64)
    with np.errstate(over="ignore"):
        return (1.0 / (1.0 + np.exp(-x))).astype(F32)


def scaled_silu(d, hc):
    """bot from bf16-valued down outputs d [M, lr]."""
    sc = round_bf16(np.asarray(d, F32) / F32(hc))
    return round_bf16(sc * sigmoid32(sc))


def gate_mean(nrm, g, hc):
    """out [M, H] from nrm [M, hc*H] and bf16-valued gate logits g [M, hc*H]."""
    nrm = np.asarray(nrm, F32)
    g = np.asarray(g, F32)
    M, n = g.shape
    H = n // hc
    gate = round_bf16(sigmoid32(g))
    term = round_bf16(nrm[:, :n] * gate)
    tot = np.zeros((M, H), F32)
    for s in range(hc):
        tot = (tot + term[:, s * H:(s + 1) * H]).astype(F32)
    return round_bf16(tot / F32(hc))


def mixer(x, qd, sd, qu, su, lr, hc):
    """Full mixer on bf16-valued x [M, hc*H]: returns (di [M, Nd], bot [M, lr],
    block_input [M, H]) with numpy fp32 GEMV sums."""
    di = gemv.w8_linear(x, qd, sd, "bf16")
    bot = scaled_silu(di[:, :lr], hc)
    g = gemv.w8_linear(bot, qu, su, "bf16")
    return di, bot, gate_mean(x, g, hc)


def interleave_up(q, s, hc, bj):
    idx = quant.interleave_up_rows(q.shape[0], hc, bj)
    return q[idx], s[idx]
