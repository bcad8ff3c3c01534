"""The draft head's oracle functions against float64 sums and invariants (CPU)."""
import numpy as np

from oracle import formats as fm
from oracle import head as oh
from oracle import ordered
from oracle import quant as oq


def _setup(seed=11, V=64, K=256, M=3, C=8):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    w[rng.integers(0, V, 4)] *= 40                      # a few rows far from the rest
    P, S, gs = oq.quantize_nv4(w)
    x = fm.round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    rows = np.stack([rng.choice(V, C, replace=False) for _ in range(M)]).astype(np.int64)
    return rng, P, S, gs, x, rows


def test_nv4_rows_within_step_bound_of_exact_sum():
    for lpr in (1, 2, 8):
        _, P, S, gs, x, rows = _setup()
        got = oh.nv4_rows(fm.bf16_bits(x), P, S, gs, rows, lpr)
        op = oq.dequant_nv4_operand(P, S)                  # exact fp32 (and bf16) operand
        assert np.array_equal(fm.round_bf16(op), op)
        for m in range(x.shape[0]):
            wr = op[rows[m]]
            exact = (x[m].astype(np.float64) @ wr.astype(np.float64).T) * float(gs)
            bound = ordered.step_bound(x[m:m + 1], wr, 32, lpr)[0] * float(gs) + np.abs(exact) * 2.0 ** -23
            assert np.all(np.abs(got[m] - exact) <= bound), (lpr, m)


def test_nv4_rows_gather_and_scale():
    rng, P, S, gs, x, rows = _setup(seed=12)
    xb = fm.bf16_bits(x)
    got = oh.nv4_rows(xb, P, S, gs, rows, 2)
    perm = rng.permutation(rows.shape[1])
    assert np.array_equal(oh.nv4_rows(xb, P, S, gs, rows[:, perm], 2), got[:, perm])
    one = oh.nv4_rows(xb, P, S, 1.0, rows, 2)
    assert np.array_equal((one * np.float32(gs)).astype(np.float32), got)   # gs: one fp32 multiply at the end
    # a row of a single nonzero code: the sum is that one exact product times gs
    P1 = np.zeros_like(P)
    P1[0, 3] = 0x20                                      # code 2 (value 1.0) at k = 7
    S1 = np.full_like(S, 0x38)                           # e4m3 1.0
    r = oh.nv4_rows(xb, P1, S1, 2.0, np.zeros((x.shape[0], 1), np.int64), 2)
    assert np.array_equal(r[:, 0], (x[:, 7] * 2.0).astype(np.float32))


def test_draft_head_scatter():
    rng = np.random.default_rng(13)
    V, K, M, dc, vocab = 96, 256, 2, 8, 300
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    P, S, gs = oq.quantize_nv4(w)
    P2, S2 = oq.quantize_int2(oq.dequant_nv4(P, S, gs), group=16)
    ids = np.sort(rng.choice(vocab, V, replace=False))
    x = fm.round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    cand, vals, full = oh.draft_head(fm.bf16_bits(x), P2, S2, 16, P, S, gs, ids, vocab, dc, 2)
    assert cand.shape == (M, dc) and len(set(cand[0].tolist())) == dc
    # candidates: the top dc of the fp32 coarse logits (int2_logits' default
    # dtype, x/fp4patch.py:313-314), not of their bf16 rounding
    co = oh.int2_coarse(fm.bf16_bits(x), P2, S2, 16)
    assert co.dtype == np.float32
    assert np.array_equal(cand, oh.topk_total_order(co, dc))
    # the temperature scales the fp32 values before the bf16 cast
    _, vals_t, full_t = oh.draft_head(fm.bf16_bits(x), P2, S2, 16, P, S, gs, ids, vocab, dc, 2, inv_t=0.625)
    assert np.array_equal(vals_t, (vals * np.float32(0.625)).astype(np.float32))
    assert np.array_equal(np.take_along_axis(full_t, ids[cand], 1), fm.bf16_bits(vals_t))
    keep = np.zeros((M, vocab), bool)
    np.put_along_axis(keep, ids[cand], True, 1)
    assert np.all(full[~keep] == 0xFF80)                 # -inf outside the candidates
    assert np.array_equal(np.take_along_axis(full, ids[cand], 1), fm.bf16_bits(vals))


def test_int2_coarse_is_rounded_exact_sum():
    """Coarse logits are the exact (float64) sum rounded once to fp32: equal
    to the fp32 rounding of a brute-force exact sum on a tiny head."""
    rng = np.random.default_rng(14)
    V, K = 24, 128
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    P, S = oq.quantize_int2(w, group=16)
    x = fm.round_bf16(rng.standard_normal((2, K)).astype(np.float32))
    got = oh.int2_coarse(fm.bf16_bits(x), P, S, 16, rows_per_chunk=7)
    op = fm.round_bf16(oq.dequant_int2(P, S))        # the bf16 operand bf16((code - 1.5) * s)
    from fractions import Fraction
    import exact_round as er
    for m in range(2):
        for v in range(V):
            ex = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(x[m], op[v]))
            assert Fraction(float(got[m, v])) == er.f32(ex), (m, v)


def test_fast_head_argmax_blocks():
    """fast_head_argmax (one coarse pass, top-C and rescore per block of rows)
    equals the argmax of fast_head's output row by row, with blocks that split
    the rows unevenly; a planted winner row is every row's argmax."""
    rng = np.random.default_rng(15)
    V, K, C, M = 2000, 256, 32, 7
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    q, s = oq.quantize_mx8(w)
    P, S = oq.quantize_int2(oq.mx8_dequant(q, s), group=16)
    xb = fm.bf16_bits(fm.round_bf16(rng.standard_normal((M, K)).astype(np.float32)))
    _, _, out = oh.fast_head(xb, P, S, 16, q, s, C, 4)
    want = np.argmax(fm.bf16_to_f32(out), -1)
    assert np.array_equal(oh.fast_head_argmax(xb, P, S, 16, q, s, C, 4, block=3), want)
    # a row aligned with x[0] wins row 0 by a wide margin
    w2 = w.copy()
    w2[123] = fm.bf16_to_f32(xb[0]) * 0.5
    q2, s2 = oq.quantize_mx8(w2)
    P2, S2 = oq.quantize_int2(oq.mx8_dequant(q2, s2), group=16)
    assert oh.fast_head_argmax(xb[:1], P2, S2, 16, q2, s2, C, 4)[0] == 123
