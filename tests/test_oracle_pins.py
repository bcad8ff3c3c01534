"""Pins of the oracle functions that no golden vector covers (CPU).

  - oracle.hc.scaled_silu / gate_mean: the rounding points of the mixer
    epilogues (x/fp4x_kernels.py:460-464, :486-493), against closed forms the
    mathematics fixes and against exact rational arithmetic with a 200-bit
    sigmoid (mpmath) over dense sweeps of bf16 inputs;
  - oracle.head.topk_total_order: against a brute-force lexicographic sort
    (torch.topk's set at x/fp4patch.py:377 and :315, with the HIP select's tie
    order);
  - oracle.ordered.ordered_gemv: against a sequential fold with exact
    rational fma steps on tiny inputs.

Each check is shown to fail on a mutant oracle (one rounding dropped, a wrong
zero or NaN rule, a different summation order), planted on the CPU.
"""
from fractions import Fraction

import mpmath
import numpy as np
import pytest
import torch

import exact_round as er
from oracle import formats as fm
from oracle import hc as ohc
from oracle import head as oh
from oracle import ordered

mpmath.mp.prec = 200


# ------------------------------------------------------------------ helpers
def test_exact_rounding_helper_matches_library_casts():
    rng = np.random.default_rng(0)
    d = np.concatenate([rng.standard_normal(400) * 10.0 ** rng.integers(-30, 30, 400),
                        rng.standard_normal(50) * 1e-40, [0.5 + 2.0 ** -25, 1.5 * 2.0 ** -140]])
    for v in d:
        assert er.f32(er.frac(v)) == er.frac(np.float32(v)), v             # float64 -> float32 (IEEE RNE)
    f = (rng.standard_normal(400) * 10.0 ** rng.integers(-20, 20, 400)).astype(np.float32)
    t = torch.from_numpy(f).to(torch.bfloat16).float().numpy()
    for v, w in zip(f, t):
        assert er.bf16(er.frac(v)) == er.frac(w), v                        # float32 -> bfloat16 (RNE)


def sigmoid_exact(q):
    """sigmoid of a rational to 200 bits, as a Fraction."""
    s = 1 / (1 + mpmath.exp(-mpmath.mpf(q.numerator) / q.denominator))
    man, exp = s.man_exp
    return Fraction(int(man)) * Fraction(2) ** int(exp) if man else Fraction(0)


def bf16_sweep(emin, emax, signs=(1, -1)):
    """Every bf16 value with exponent in [emin, emax] (and zero)."""
    vals = [0.0]
    for e in range(emin, emax + 1):
        for m in range(128):
            for s in signs:
                vals.append(s * (1 + m / 128) * 2.0 ** e)
    return np.array(vals, np.float32)


_SIG = {}


def sig_f32(v):
    """fp32 sigmoid of a bf16 value, correctly rounded."""
    r = _SIG.get(float(v))
    if r is None:
        r = _SIG[float(v)] = er.f32(sigmoid_exact(er.frac(v)))
    return r


def brute_scaled_silu(d, hc):
    """sc = bf16(fp32(d / hc)); bot = bf16(fp32(sc * fp32(sigmoid(sc))))."""
    out = np.empty(d.shape, np.float32)
    for i, v in np.ndenumerate(d):
        sc = er.bf16(er.f32(er.frac(v) / hc))
        out[i] = float(er.bf16(er.f32(sc * sig_f32(float(sc)))))
    return out


def brute_gate_mean(nrm, g, hc):
    """gate = bf16(fp32 sigmoid(g)); term_s = bf16(fp32(nrm_s * gate_s));
    out = bf16(fp32(fp32 sum of the terms in stream order / hc))."""
    M, n = g.shape
    H = n // hc
    out = np.empty((M, H), np.float32)
    for m in range(M):
        for j in range(H):
            tot = None
            for s in range(hc):
                gate = er.bf16(sig_f32(g[m, s * H + j]))
                term = er.bf16(er.f32(er.frac(nrm[m, s * H + j]) * gate))
                tot = term if tot is None else er.f32(tot + term)
            out[m, j] = float(er.bf16(er.f32(tot / hc)))
    return out


class SkipRound:
    """A mutant of oracle.hc.round_bf16 that returns its argument unrounded on
    the skip-th call of each oracle call (calls counted from 0)."""

    def __init__(self, skip):
        self.skip, self.n = skip, 0

    def __call__(self, f):
        i, self.n = self.n, self.n + 1
        return np.asarray(f, np.float32) if i == self.skip else fm.round_bf16(f)


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32), np.asarray(b, np.float32))


# ------------------------------------------------------------------ scaled SiLU
def silu_closed_forms(f):
    """Closed forms of bot = bf16(sc * sigmoid(sc)), sc = bf16(d / hc)."""
    # sigmoid(0) = 1/2 exactly: bot(0) = 0
    assert _same(f(np.zeros((1, 4), np.float32), 4), np.zeros((1, 4)))
    # fp32 sigmoid(x) is exactly 1 for x >= 18 (e^-18 < 2^-25, half an ulp
    # below 1) but not at 17 (e^-17 > 2^-25): there bot = sc = bf16(d / hc)
    assert ohc.sigmoid32(18.0) == 1.0 and ohc.sigmoid32(17.0) == np.float32(1 - 2.0 ** -24)
    d = np.array([[64.25, 72.5, 100.75, 3001.0]], np.float32)            # d / 3 >= 21, not bf16
    want = fm.round_bf16((d / np.float32(3)).astype(np.float32))
    assert _same(f(d, 3), want)
    # sigmoid(x) < 2^-150 for x <= -104 (e^-104 < 2^-150): fp32 0, bot = -0
    assert _same(f(np.array([[-416.0, -1024.0]], np.float32), 4), np.zeros((1, 2)))
    # x = 2, hc = 1: sc = 2, sigmoid(2) = 0.880797077977882..., fp32
    # 0.88079708814620971679688, 2 * that = 1.76159417629241943 -> bf16 1.7578125
    assert _same(f(np.array([[2.0]], np.float32), 1), [[1.7578125]])


def test_scaled_silu_closed_forms():
    silu_closed_forms(ohc.scaled_silu)


@pytest.mark.parametrize("hc", [4, 3])
def test_scaled_silu_exact_sweep(hc):
    """Every bf16 input of exponent -20..20, both signs: bit for bit."""
    d = bf16_sweep(-20, 20)[None, :]
    assert _same(ohc.scaled_silu(d, hc), brute_scaled_silu(d, hc))


@pytest.mark.parametrize("skip", [0, 1])
def test_scaled_silu_mutants_fail(monkeypatch, skip):
    """Dropping sc's rounding (call 0) or bot's (call 1) breaks the sweep
    (hc = 3: d / 3 is rarely a bf16 value)."""
    d = bf16_sweep(-3, 3)[None, :]
    want = brute_scaled_silu(d, 3)
    mut = SkipRound(skip)

    def mutant(dd, hc):
        mut.n = 0
        return ohc.scaled_silu(dd, hc)

    monkeypatch.setattr(ohc, "round_bf16", mut)
    assert not _same(mutant(d, 3), want)
    if skip == 1:
        with pytest.raises(AssertionError):
            silu_closed_forms(mutant)


# ------------------------------------------------------------------ gate mean
def gate_closed_forms(f):
    # gate = 1 for g >= 18: out = bf16(sum_s nrm_s / hc); with 4 streams
    # 1 + 1.0078125 + 1 + 1 = 4.0078125, / 4 = 1 + 2^-9 -> bf16 1.0
    nrm = np.array([[1.0, 1.0078125, 1.0, 1.0]], np.float32)
    assert _same(f(nrm, np.full((1, 4), 18.0, np.float32), 4), [[1.0]])
    # gate = 0 for g <= -104 (fp32 sigmoid underflows to 0): out = 0
    assert _same(f(nrm, np.full((1, 4), -104.0, np.float32), 4), [[0.0]])
    # g = 0: gate = 1/2, terms nrm / 2 are exact: out = bf16(sum nrm / 8)
    nrm2 = np.array([[3.0, 5.0, 1.5, 0.25]], np.float32)
    assert _same(f(nrm2, np.zeros((1, 4), np.float32), 4), [[1.21875]])      # 9.75 / 8 exactly
    # g = 1 with one stream: gate = bf16(0.7310585786...) = 187/256; term =
    # bf16(1.0078125 * 187/256) = bf16(24123/32768) = 188/256
    assert _same(f(np.array([[1.0078125]], np.float32), np.ones((1, 1), np.float32), 1), [[188 / 256]])


def test_gate_mean_closed_forms():
    gate_closed_forms(ohc.gate_mean)


@pytest.mark.parametrize("hc", [4, 3])
def test_gate_mean_exact_sweep(hc):
    """Gate logits over every bf16 value of exponent -8..7, random bf16
    normalized inputs: bit for bit."""
    rng = np.random.default_rng(hc)
    g = bf16_sweep(-8, 7)
    H = -(-g.size // hc)
    g = np.resize(g, hc * H)[None, :]
    nrm = fm.round_bf16((rng.standard_normal(hc * H) * 2).astype(np.float32))[None, :]
    assert _same(ohc.gate_mean(nrm, g, hc), brute_gate_mean(nrm, g, hc))


@pytest.mark.parametrize("skip", [0, 1, 2])
def test_gate_mean_mutants_fail(monkeypatch, skip):
    """Dropping the gate's (call 0), the terms' (call 1) or the output's
    (call 2) bf16 rounding breaks the sweep."""
    rng = np.random.default_rng(7)
    g = bf16_sweep(-4, 3)
    H = g.size // 4
    g = g[:4 * H][None, :]
    nrm = fm.round_bf16((rng.standard_normal(4 * H) * 2).astype(np.float32))[None, :]
    want = brute_gate_mean(nrm, g, 4)
    mut = SkipRound(skip)

    def mutant(n, gg, hc):
        mut.n = 0
        return ohc.gate_mean(n, gg, hc)

    monkeypatch.setattr(ohc, "round_bf16", mut)
    assert not _same(mutant(nrm, g, 4), want)
    if skip == 2:
        with pytest.raises(AssertionError):
            gate_closed_forms(mutant)


def test_sigmoid32_correctly_rounded():
    """oracle.hc.sigmoid32 (float64 exp, rounded to fp32) equals the
    correctly rounded fp32 sigmoid on every bf16 input of exponent -12..7."""
    x = bf16_sweep(-12, 7)
    got = ohc.sigmoid32(x)
    for v, s in zip(x, got):
        assert er.frac(s) == sig_f32(float(v)), v


# ------------------------------------------------------------------ top-k order
def brute_topk(vals, C):
    """Indices of the C largest per row by (value desc, index asc), -0 == +0,
    NaN above everything: a stable lexicographic sort on (NaN flag, value)
    with the index as the last key."""
    f = vals.astype(np.float64) if vals.dtype == np.float32 else fm.bf16_to_f32(vals).astype(np.float64)
    out = []
    for row in f:
        nan = np.isnan(row)
        v = np.where(nan, 0.0, row)
        order = np.lexsort((np.arange(row.size), -v, -nan.astype(np.int64)))
        out.append(order[:C])
    return np.array(out, np.int64)


def topk_rows_cases():
    rng = np.random.default_rng(5)
    bits = fm.bf16_bits((rng.standard_normal((4, 300)) * 3).astype(np.float32))
    bits[1] = fm.bf16_bits(np.round(fm.bf16_to_f32(bits[1])))                 # heavy ties
    bits[2, :9] = [0x8000, 0x0000, 0x7FC0, 0xFF80, 0x7F80, 0xFFC1, 0x0001, 0x8001, 0x8000]
    bits[3, :] = 0x8000
    bits[3, ::7] = 0x0000                                                     # all zeros, both signs
    bits[3, 100:104] = [0x7FC0, 0x7F81, 0xFFFF, 0x7FC0]                       # NaNs of several payloads
    f = (rng.standard_normal((3, 500)) * 2).astype(np.float32)
    f[1] = np.round(f[1])
    f[2, :8] = [-0.0, 0.0, np.nan, -np.inf, np.inf, -np.nan, 1e-45, -1e-45]
    return bits, f


@pytest.mark.parametrize("C", [1, 7, 64, 300])
def test_topk_total_order_brute_force(C):
    bits, f = topk_rows_cases()
    assert np.array_equal(oh.topk_total_order(bits, C), brute_topk(bits, C))
    if C <= 300:
        assert np.array_equal(oh.topk_total_order(f, min(C, 500)), brute_topk(f, min(C, 500)))


def test_topk_mutants_fail(monkeypatch):
    bits, f = topk_rows_cases()
    want_b, want_f = brute_topk(bits, 64), brute_topk(f, 64)
    real = oh.order_keys

    def no_zero_fold(v):                       # -0 ranked below +0
        a = np.asarray(v)
        k = real(v)
        neg0 = (a == 0x8000) if a.dtype == np.uint16 else ((a == 0) & np.signbit(a))
        return np.where(neg0, k - 1, k)

    def nan_smallest(v):
        a = np.asarray(v)
        k = real(v)
        nan = fm.bf16_to_f32(a) if a.dtype == np.uint16 else a
        return np.where(np.isnan(nan), 0, k)

    for mut in (no_zero_fold, nan_smallest):
        monkeypatch.setattr(oh, "order_keys", mut)
        assert not (np.array_equal(oh.topk_total_order(bits, 64), want_b)
                    and np.array_equal(oh.topk_total_order(f, 64), want_f)), mut.__name__
    monkeypatch.setattr(oh, "order_keys", real)


# ------------------------------------------------------------------ ordered fma sums
def fold_exact(x, w, kpc, lpr, ksplit, gs):
    """The rescore order, every step an exact rational rounded once to fp32."""
    M, K = x.shape
    N = w.shape[0]
    ks = K // ksplit
    chunks = ks // kpc
    out = np.empty((M, N), np.float32)
    for m in range(M):
        for n in range(N):
            tot = None
            for s in range(ksplit):
                v = []
                for l in range(lpr):
                    acc = Fraction(0)
                    for c in range(l, chunks, lpr):
                        for k in range(s * ks + c * kpc, s * ks + (c + 1) * kpc):
                            acc = er.f32(er.frac(w[n, k]) * er.frac(x[m, k]) + acc)
                    v.append(acc)
                st = 1
                while st < lpr:
                    v = [er.f32(v[l] + v[l ^ st]) for l in range(lpr)]
                    st <<= 1
                p = er.f32(v[0] * er.frac(np.float32(gs)))
                tot = p if tot is None else er.f32(tot + p)
            out[m, n] = float(tot)
    return out


def fold_inputs(seed):
    """bf16 operands spanning 2^-20 .. 2^20, so the summation order matters."""
    rng = np.random.default_rng(seed)
    K = 128
    x = fm.round_bf16((rng.standard_normal((2, K)) * 2.0 ** rng.integers(-10, 10, (2, K))).astype(np.float32))
    w = fm.round_bf16((rng.standard_normal((3, K)) * 2.0 ** rng.integers(-10, 10, (3, K))).astype(np.float32))
    return x, w


@pytest.mark.parametrize("kpc,lpr,ksplit,gs", [(16, 1, 1, 1.0), (16, 4, 1, 1.0), (32, 2, 2, 0.3719),
                                              (16, 8, 1, 2.5)])
def test_ordered_gemv_exact_fold(kpc, lpr, ksplit, gs):
    x, w = fold_inputs(kpc + lpr)
    got = ordered.ordered_gemv(fm.bf16_bits(x), fm.bf16_bits(w), kpc, lpr, ksplit=ksplit, gs=gs)
    assert _same(got, fold_exact(x, w, kpc, lpr, ksplit, gs))


def test_ordered_gemv_order_is_observable():
    """A different lane split of the same sum gives different bits on these
    inputs: the fold above pins the order, not only the value."""
    x, w = fold_inputs(3)
    a = ordered.ordered_gemv(fm.bf16_bits(x), fm.bf16_bits(w), 16, 4)
    b = fold_exact(x, w, 16, 1, 1, 1.0)
    c = fold_exact(x, w, 16, 2, 1, 1.0)
    assert not _same(a, b) and not _same(a, c)
    # and every order stays within the step bound of the exact sum
    exact = ordered.exact_sum(x, w)
    assert np.all(np.abs(a - exact) <= ordered.step_bound(x, w, 16, 4))
