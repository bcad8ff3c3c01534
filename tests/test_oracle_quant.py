"""Oracle quantizers pinned against the reference's own golden vectors
(tests/golden/make_golden.py) and invariants; the product's torch weight
preparation checked against the oracle."""
import numpy as np
import pytest
import torch

from oracle import formats as fm
from oracle import quant as oq
from oracle import hc as ohc


def test_w8_golden(golden):
    q, s = oq.quantize_w8(golden["w8_w"])
    assert np.array_equal(q, golden["w8_q"])
    assert np.array_equal(s.view(np.uint32), golden["w8_s"].view(np.uint32))
    # tie row: values at .5 steps of a power-of-two scale round half to even
    assert list(q[7, :9]) == [127, 2, -4, 0, 0, 2, 126, -126, 64]


def test_w6_golden(golden):
    L, H, S = oq.quantize_w6(golden["w6_w"])
    assert np.array_equal(L, golden["w6_L"]) and np.array_equal(H, golden["w6_H"])
    assert np.array_equal(S.view(np.uint16), golden["w6_S"].view(np.uint16))
    codes = oq.w6_codes(L, H) - 32
    assert list(codes[7, :8]) == [31, 2, -4, 30, -30, 0, 0, 8]
    assert list(codes[7, 32:36]) == [-31, -30, 2, -2]


def test_w6_clip_search_golden(golden):
    L, H, S = oq.quantize_w6(golden["w6_w"], qmax=15, clip_search=3)
    assert np.array_equal(L, golden["w6c_L"]) and np.array_equal(H, golden["w6c_H"])
    assert np.array_equal(S.view(np.uint16), golden["w6c_S"].view(np.uint16))


def test_w6_clip_grid_and_sum_order():
    """The clip search's two fp32 details, pinned against torch's own CPU
    results: clip_grid(n) is torch.linspace(0.70, 0.98, n) for n = 1..64
    (numpy's float64 linspace rounded to fp32 differs from n = 3 on), and
    sum_sq32 is torch's fp32 sum of the squares over a 32-element row, here on
    magnitudes over 12 decades (a sequential or pairwise sum differs on most
    such rows)."""
    for n in range(1, 65):
        want = np.array(torch.linspace(0.70, 0.98, n).tolist(), np.float32)
        assert np.array_equal(np.array(oq.clip_grid(n), np.float32), want), n
    rng = np.random.default_rng(9)
    d = (rng.standard_normal((4096, 32)) * 10.0 ** rng.uniform(-6, 6, (4096, 32))).astype(np.float32)
    want = (torch.from_numpy(d) ** 2).sum(-1, keepdim=True).numpy()
    assert np.array_equal(oq.sum_sq32(d).view(np.uint32), want.view(np.uint32))
    seq = (d * d)[:, :1].copy()
    for i in range(1, 32):
        seq = seq + (d * d)[:, i:i + 1]
    assert (seq != want).mean() > 0.3                     # the order matters on these rows


@pytest.mark.parametrize("qmax,clip", [(31, 3), (15, 7), (31, 16), (7, 1)])
def test_w6_clip_search_torch_formulas(qmax, clip):
    """The oracle's clip search equals the reference's torch formulas (the
    product's CPU fallback of quantize_w6) bit for bit on N(0, 0.02) rows,
    rows with one outlier per group, and rows of values on the W6 grid."""
    import fp4x_kernels as F
    rng = np.random.default_rng(qmax + clip)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    w[:8, ::32] *= 20
    w[8:16] = (rng.integers(-qmax, qmax + 1, (8, 256)) * np.float32(2.0 ** -7)).astype(np.float32)
    got = F.quantize_w6(torch.from_numpy(w), qmax, clip)
    want = oq.quantize_w6(w, qmax, clip)
    for g, t in zip(got, want):
        assert np.array_equal(g.numpy().view(np.uint8), np.asarray(t).view(np.uint8))
    plain = oq.quantize_w6(w, qmax)
    assert not np.array_equal(want[2], plain[2])          # the search moved some scales


def test_mx8_dequant_golden(golden):
    got = oq.mx8_dequant(golden["mx8_w"], golden["mx8_s"])
    assert np.array_equal(got.view(np.uint32), golden["mx8_deq"].view(np.uint32))


def test_nv4_golden(golden):
    P, S, gs = oq.quantize_nv4(golden["nv4_w"])
    assert gs == float(golden["nv4_gs"])
    assert np.array_equal(P, golden["nv4_P"]) and np.array_equal(S, golden["nv4_S"])
    deq = oq.dequant_nv4(P, S, gs)
    assert np.array_equal(deq.view(np.uint32), golden["nv4_deq"].view(np.uint32))


@pytest.mark.parametrize("grp", [16, 32])
def test_int2_golden(golden, grp):
    P, S = oq.quantize_int2(golden["int2_w"], group=grp)
    assert np.array_equal(P, golden[f"int2g{grp}_P"])
    assert np.array_equal(S.view(np.uint16), golden[f"int2g{grp}_S"].view(np.uint16))
    deq = oq.dequant_int2(P, S)
    assert np.array_equal(deq.view(np.uint32), golden[f"int2g{grp}_deq"].view(np.uint32))


def test_int2_e4m3_golden(golden):
    P, S, R = oq.quantize_int2(golden["int2_w"], scale_fmt="e4m3", group=16)
    assert np.array_equal(P, golden["int2e_P"]) and np.array_equal(S, golden["int2e_S"])
    assert np.array_equal(R.view(np.uint32), golden["int2e_R"].view(np.uint32))


def test_interleave_golden(golden):
    idx = oq.interleave_up_rows(32, 4, 2)
    assert np.array_equal(golden["il_q"][idx], golden["il_qi"])


# ---------------------------------------------------------------- invariants
def test_w8_invariants():
    w = np.random.default_rng(3).standard_normal((16, 256)).astype(np.float32) * 0.02
    q, s = oq.quantize_w8(w)
    err = np.abs(oq.dequant_w8(q, s) - w).reshape(16, 4, 64)
    assert np.all(err <= s[..., None] * 0.5000001)
    assert np.abs(q.astype(np.int32)).max() == 127


def test_w6_layout_roundtrip():
    rng = np.random.default_rng(4)
    codes = rng.integers(0, 64, (8, 64)).astype(np.int32)
    lo, hi = codes & 15, codes >> 4
    L = (lo[:, 0::2] | (lo[:, 1::2] << 4)).astype(np.uint8)
    H = (hi[:, 0::4] | (hi[:, 2::4] << 2) | (hi[:, 1::4] << 4) | (hi[:, 3::4] << 6)).astype(np.uint8)
    assert np.array_equal(oq.w6_codes(L, H), codes)
    # the hi bits of k%4 = 0, 2, 1, 3 occupy bit pairs 0, 1, 2, 3
    assert oq.w6_codes(np.zeros((1, 2), np.uint8), np.array([[0b11_01_10_00]], np.uint8))[0].tolist() == \
        [0, 1 << 4, 2 << 4, 3 << 4]


def test_int2_order_and_levels():
    P = np.array([[0b11_01_10_00]], np.uint8)   # bit pairs 0..3 hold codes 0, 2, 1, 3
    assert oq.int2_codes(P)[0].tolist() == [0, 1, 2, 3]   # element j in bit pair ORDER[j]
    w = np.random.default_rng(5).standard_normal((4, 64)).astype(np.float32)
    P, S = oq.quantize_int2(w)
    err = np.abs(oq.dequant_int2(P, S) - w).reshape(4, 4, 16)
    assert np.all(err <= S.astype(np.float32)[..., None] * 1.0 + 1e-6)


def test_mx8_quantizer_ocp_rules():
    rng = np.random.default_rng(6)
    w = rng.standard_normal((8, 128)).astype(np.float32) * 0.02
    w[0, :32] = 0.0
    q, s = oq.quantize_mx8(w)
    amax = np.abs(w.reshape(8, 4, 32)).max(-1)
    nz = amax > 0
    assert np.array_equal(s[nz].astype(np.int64) - 127, np.floor(np.log2(amax[nz])).astype(np.int64) - 8)
    assert s[0, 0] == 0
    deq = oq.mx8_dequant(q, s)
    X = np.exp2(s.astype(np.float64) - 127).repeat(32, 1)
    v = w / X                                   # element in units of the shared scale, |v| < 512
    d = deq / X
    sat = np.abs(v) >= 448
    assert np.all(d[sat] == np.sign(v[sat]) * 448)
    normal = ~sat & (np.abs(v) >= 2.0 ** -6)
    assert np.all(np.abs(d - v)[normal] <= np.abs(v)[normal] * 2.0 ** -4)   # half an e4m3 ulp
    sub = np.abs(v) < 2.0 ** -6
    assert np.all(np.abs(d - v)[sub] <= 2.0 ** -10)                         # half a subnormal step


def test_nv4_invariants():
    w = np.random.default_rng(7).standard_normal((8, 64)).astype(np.float32) * 0.02
    P, S, gs = oq.quantize_nv4(w)
    assert np.all(np.isin(oq.nv4_values(P), fm.E2M1))
    assert gs == max(float(np.abs(w).max()) / 6.0 / 448.0, 1e-30)


# ---------------------------------------------------------------- product weight prep
@pytest.fixture(scope="module")
def F():
    import fp4x_kernels
    return fp4x_kernels


def test_product_quantizers_match_oracle(F, golden):
    w = torch.from_numpy(golden["w8_w"])
    q, s = F.quantize_w8(w)
    assert np.array_equal(q.numpy(), golden["w8_q"]) and np.array_equal(s.numpy(), golden["w8_s"])
    L, H, S = F.quantize_w6(torch.from_numpy(golden["w6_w"]))
    assert np.array_equal(L.numpy(), golden["w6_L"]) and np.array_equal(H.numpy(), golden["w6_H"])
    assert np.array_equal(S.numpy().view(np.uint16), golden["w6_S"].view(np.uint16))
    L, H, S = F.quantize_w6(torch.from_numpy(golden["w6_w"]), 15, 3)
    assert np.array_equal(L.numpy(), golden["w6c_L"]) and np.array_equal(S.numpy(), golden["w6c_S"])
    P, S, gs = F.quantize_nv4(torch.from_numpy(golden["nv4_w"]))
    assert np.array_equal(P.numpy(), golden["nv4_P"]) and gs == float(golden["nv4_gs"])
    assert np.array_equal(S.view(torch.uint8).numpy(), golden["nv4_S"])
    assert np.array_equal(F.dequant_nv4(P, S, gs).numpy(), golden["nv4_deq"])
    for grp in (16, 32):
        P, S = F.quantize_int2(torch.from_numpy(golden["int2_w"]), group=grp)
        assert np.array_equal(P.numpy(), golden[f"int2g{grp}_P"])
        assert np.array_equal(F.dequant_int2(P, S).numpy(), golden[f"int2g{grp}_deq"])
    P, S, R = F.quantize_int2(torch.from_numpy(golden["int2_w"]), scale_fmt="e4m3")
    assert np.array_equal(S.view(torch.uint8).numpy(), golden["int2e_S"]) and np.array_equal(R.numpy(), golden["int2e_R"])
    qi, si = F.HCFused.interleave_up(torch.from_numpy(golden["il_q"]), torch.arange(32.).view(32, 1), 4, 2)
    assert np.array_equal(qi.numpy(), golden["il_qi"])


def test_product_mx8_quantizer_matches_oracle(F):
    rng = np.random.default_rng(8)
    w = rng.standard_normal((16, 256)).astype(np.float32) * 0.02
    w[1, :32] = 0
    w[2, 32:64] *= 1e5
    w[3, :32] = 1e-41      # fp32 subnormal block
    q, s = F.quantize_mx8(torch.from_numpy(w))
    oq_q, oq_s = oq.quantize_mx8(w)
    assert np.array_equal(s.numpy(), oq_s)
    assert np.array_equal(q.numpy(), oq_q)


def test_hc_oracle_closed_forms():
    # sigmoid(0) = 1/2: silu(0) = 0; gate-mean of equal streams is the stream value times the gate
    assert ohc.scaled_silu(np.zeros((1, 4), np.float32), 4).tolist() == [[0.0] * 4]
    nrm = np.full((1, 8), 2.0, np.float32)
    g = np.zeros((1, 8), np.float32)
    assert ohc.gate_mean(nrm, g, 4).tolist() == [[1.0, 1.0]]


def nv4_midpoint_case(seed=0):
    """A [2, 16] matrix whose row 0 holds, besides its scale-setting maximum,
    elements w with fp32(w / sf) exactly on an e2m1 midpoint while the exact
    quotient lies above it: fp32 and fp64 evaluation of the reference's
    v = w / (sc.float() * gs) disagree on those elements' magnitude."""
    rng = np.random.default_rng(seed)
    mids = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    while True:
        big = np.float32(rng.uniform(1.0, 2.0))
        amax = np.float32(big * np.float32(rng.uniform(0.05, 0.9)))
        w = np.zeros((2, 16), np.float32)
        w[1, 0] = big                                             # the global maximum (sets gs)
        w[0, 0] = amax
        gs = max(float(big) / 6.0 / 448.0, 1e-30)
        sc = np.clip(amax / np.float32(6.0) / np.float32(gs), np.float32(2.0 ** -9), np.float32(448.0))
        sf = np.float32(fm.e4m3_decode(fm.e4m3_encode(np.array([sc])))[0] * np.float32(gs))
        hits = []
        for m in mids:
            f = np.float32(np.float64(m) * np.float64(sf))
            if f < amax and np.float32(f / sf) == np.float32(m) and np.float64(f) / np.float64(sf) > m:
                hits.append(f)
        if len(hits) >= 2:
            w[0, 1:1 + len(hits)] = hits
            return w, len(hits)


def test_nv4_quotient_is_fp32():
    """The oracle follows the reference's fp32 ops: sf = fp32(sc * gs) and v =
    fp32(w / sf); ties at a midpoint round down.  Pinned against torch on CPU
    evaluating the reference's expression (x/fp4x_kernels.py:293-296)."""
    w, n = nv4_midpoint_case()
    P, S, gs = oq.quantize_nv4(w)
    nib = oq.nv4_values(P)[0, 1:1 + n]
    g = torch.from_numpy(w).reshape(2, 1, 16)
    sc = (g.abs().amax(-1, keepdim=True) / 6.0 / gs).clamp(min=2 ** -9, max=448.0).to(torch.float8_e4m3fn)
    lut = torch.tensor([0, .5, 1, 1.5, 2, 3, 4, 6])
    v = (g / (sc.float() * gs)).clamp(-6, 6)
    want = lut[torch.bucketize(v.abs(), (lut[1:] + lut[:-1]) / 2)].reshape(2, 16)[0, 1:1 + n].numpy()
    assert np.array_equal(nib, want)
    # the same elements evaluated in fp64 land one level higher
    sf64 = fm.e4m3_decode(S[0, 0]) * np.float64(np.float32(gs))
    up = np.searchsorted(oq._MIDS, np.abs(w[0, 1:1 + n].astype(np.float64) / sf64), side="left")
    assert np.all(fm.E2M1[up] > nib)
