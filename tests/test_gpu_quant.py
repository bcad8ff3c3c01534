"""Weight preparation on the GPU (csrc/fp4x_quant.hip): the HIP quantizers
equal the oracle's quantizers bit for bit (codes, scales, the NVFP4 global
scale, the e4m3 INT2 row scales) for fp32, bf16, MXFP8 and NVFP4 sources, on the reference's golden
vectors, on random matrices with degenerate groups, and on the NVFP4
midpoint case where fp32 and fp64 evaluation differ."""
import numpy as np
import pytest
import torch

from oracle import formats as fm
from oracle import quant as oq

from gpu_helpers import dev
from test_oracle_quant import nv4_midpoint_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def F():
    import fp4x_kernels
    return fp4x_kernels


def np_(t):
    if t.dtype == torch.float8_e4m3fn:
        t = t.view(torch.uint8)
    return t.cpu().numpy()


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype.kind == "f":
        a = a.view(np.uint32 if a.itemsize == 4 else np.uint16)
    if b.dtype.kind == "f":
        b = b.view(np.uint32 if b.itemsize == 4 else np.uint16)
    return a.shape == b.shape and np.array_equal(a, b)


def check(fmt, got, w, group=16, qmax=31):
    """got (device tuple) against the oracle quantizer of fp32 weights w
    (fmt "int2e": INT2 with e4m3 group scales and fp32 row scales)."""
    if fmt == "w8":
        want = oq.quantize_w8(w)
    elif fmt == "w6":
        want = oq.quantize_w6(w, qmax)
    elif fmt == "nv4":
        want = oq.quantize_nv4(w)
        assert got[2] == want[2], (got[2], want[2])                # gs, the python float
        got, want = got[:2], want[:2]
    elif fmt == "int2e":
        want = oq.quantize_int2(w, scale_fmt="e4m3", group=group)
    else:
        want = oq.quantize_int2(w, group=group)
    assert len(got) == len(want)
    for i, (g, t) in enumerate(zip(got, want)):
        assert same(np_(g), t), (fmt, i, int((np_(g).reshape(-1) != np.asarray(t).reshape(-1)).sum()))


def test_golden_vectors(gpu, F, golden):
    q, s = F.quantize_w8(dev(golden["w8_w"]))
    assert same(np_(q), golden["w8_q"]) and same(np_(s), golden["w8_s"])
    L, H, S = F.quantize_w6(dev(golden["w6_w"]))
    assert same(np_(L), golden["w6_L"]) and same(np_(H), golden["w6_H"]) and same(np_(S), golden["w6_S"])
    L, H, S = F.quantize_w6(dev(golden["w6_w"]), 15, 3)                   # with the clip search
    assert same(np_(L), golden["w6c_L"]) and same(np_(H), golden["w6c_H"]) and same(np_(S), golden["w6c_S"])
    P, S, gs = F.quantize_nv4(dev(golden["nv4_w"]))
    assert same(np_(P), golden["nv4_P"]) and same(np_(S), golden["nv4_S"]) and gs == float(golden["nv4_gs"])
    for grp in (16, 32):
        P, S = F.quantize_int2(dev(golden["int2_w"]), group=grp)
        assert same(np_(P), golden[f"int2g{grp}_P"]) and same(np_(S), golden[f"int2g{grp}_S"])
    P, S, R = F.quantize_int2(dev(golden["int2_w"]), scale_fmt="e4m3", group=16)
    assert S.dtype == torch.float8_e4m3fn and R.dtype == torch.float32 and R.shape == (golden["int2_w"].shape[0],)
    assert same(np_(P), golden["int2e_P"]) and same(np_(S), golden["int2e_S"]) and same(np_(R), golden["int2e_R"])


def weights(seed, n=384, k=2560):
    """N(0, 0.02) rows with degenerate and tie groups: a zero row, a row of
    1e-9 (INT2 scales that underflow fp16), a row of 1e3, values on the .5
    ties of the W8 and W6 grids, and a row mixing +-0."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[1] = 0
    w[2] = (rng.standard_normal(k) * 1e-9).astype(np.float32)
    w[3] *= 5e4
    s8 = np.float32(2.0 ** -6)
    w[4] = (rng.integers(-126, 127, k) + 0.5).astype(np.float32) * s8
    w[4, ::64] = 127 * s8                                              # scale s8 exactly
    w[5] = (rng.integers(-30, 31, k) + 0.5).astype(np.float32) * np.float32(2.0 ** -8)
    w[5, ::32] = 31 * np.float32(2.0 ** -8)
    w[6] = np.where(rng.random(k) < 0.5, np.float32(0.0), np.float32(-0.0))
    w[6, 100] = 0.5
    return w


@pytest.mark.parametrize("fmt", ["w8", "w6", "nv4", "int2", "int2e"])
@pytest.mark.parametrize("src", ["f32", "bf16"])
def test_dense_sources(gpu, F, fmt, src):
    w = weights(11)
    if src == "bf16":
        w = fm.round_bf16(w)
        t = dev(fm.bf16_bits(w).view(np.int16)).view(torch.bfloat16)
    else:
        t = dev(w)
    if fmt == "w8":
        got = F.quantize_w8(t)
    elif fmt == "w6":
        got = F.quantize_w6(t)
        check("w6", F.quantize_w6(t, 15), w, qmax=15)
    elif fmt == "nv4":
        got = F.quantize_nv4(t)
    elif fmt == "int2e":
        for grp in (32, 64):
            check(fmt, F.quantize_int2(t, scale_fmt="e4m3", group=grp), w, group=grp)
        got = F.quantize_int2(t, scale_fmt="e4m3", group=16)
    else:
        for grp in (32, 64):
            check("int2", F.quantize_int2(t, group=grp), w, group=grp)
        got = F.quantize_int2(t, group=16)
    check(fmt, got, w)


def test_int2e_scale_edges(gpu, F):
    """e4m3 INT2 groups at the ends of the scale range: groups 2^-20 and
    2^-21 times the row's largest (s / rs rounds to e4m3 0: sf = 0, codes
    3 / 0 / 0 for positive, negative and zero elements), groups whose s / rs
    sits near the e4m3 subnormal ties (i + 1/2) 2^-9, zero groups beside 0.5,
    a zero row, and each row's largest group (s / rs = 448 up to one fp32
    rounding)."""
    k = 256
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((8, k)) * 0.02).astype(np.float32)
    w[0, :16] = 1.0
    w[0, 16:32] = np.float32(2.0 ** -20) * np.sign(rng.standard_normal(16)).astype(np.float32)
    w[0, 32:48] = 0
    w[0, 40] = np.float32(2.0 ** -21)
    for i in range(8):                                  # amax / row amax = (i + 1/2) 2^-9 / 448
        g = w[1, 16 * (i + 1):16 * (i + 2)]
        w[1, 16 * (i + 1):16 * (i + 2)] = g * (np.float32((i + 0.5) * 2.0 ** -9 / 448) / np.abs(g).max())
    w[1, :16] = 1.0
    w[2] = np.where(rng.random(k) < 0.5, np.float32(0.0), np.float32(-0.0))
    w[2, 100] = 0.5
    w[3] = 0
    check("int2e", F.quantize_int2(dev(w), scale_fmt="e4m3"), w)


@pytest.mark.parametrize("fmt", ["w8", "w6", "nv4", "int2", "int2e"])
def test_packed_sources(gpu, F, fmt):
    """requantize_mx8 / requantize_nv4 equal the quantizer of the packed rows'
    exact dequant (the plugin's layer, LM-head and draft-head preparation;
    int2e: INT2 with e4m3 group scales and fp32 row scales)."""
    w = weights(12)
    kw = {"scale_fmt": "e4m3"} if fmt == "int2e" else {}
    f = "int2" if fmt == "int2e" else fmt
    q8, s8 = oq.quantize_mx8(w)
    got = F.requantize_mx8(dev(q8), dev(s8), f, **kw)
    check(fmt, got, oq.mx8_dequant(q8, s8))
    P, S, gs = oq.quantize_nv4(w)
    got = F.requantize_nv4(dev(P), dev(S).view(torch.float8_e4m3fn), gs, f, **kw)
    check(fmt, got, oq.dequant_nv4(P, S, gs))


@pytest.mark.parametrize("qmax,clip", [(31, 3), (15, 7), (31, 16)])
def test_w6_clip_search(gpu, F, qmax, clip):
    """quantize_w6 with the clip search equals the oracle's bit for bit, from
    fp32 and bf16 rows and from packed MXFP8 rows (the plugin's dense layer
    preparation under FP4X_DENSE_CLIP)."""
    w = weights(13 + clip)
    w[8:16, ::32] *= 20                                     # one outlier per group: the search clips it
    got = F.quantize_w6(dev(w), qmax, clip)
    want = oq.quantize_w6(w, qmax, clip)
    for i, (g, t) in enumerate(zip(got, want)):
        assert same(np_(g), t), ("w6 clip", i, int((np_(g).reshape(-1) != np.asarray(t).reshape(-1)).sum()))
    wb = fm.round_bf16(w)
    got = F.quantize_w6(dev(fm.bf16_bits(wb).view(np.int16)).view(torch.bfloat16), qmax, clip)
    for g, t in zip(got, oq.quantize_w6(wb, qmax, clip)):
        assert same(np_(g), t)
    q8, s8 = oq.quantize_mx8(w)
    got = F.requantize_mx8(dev(q8), dev(s8), "w6", qmax=qmax, clip_search=clip)
    for g, t in zip(got, oq.quantize_w6(oq.mx8_dequant(q8, s8), qmax, clip)):
        assert same(np_(g), t)


def test_nv4_midpoints(gpu, F):
    """Elements whose fp32 quotient sits exactly on an e2m1 midpoint: the
    kernel evaluates in fp32 and rounds the tie down, as the reference does."""
    w, _ = nv4_midpoint_case()
    w = np.concatenate([w, np.zeros((2, 48), np.float32)], 1)       # K = 64
    check("nv4", F.quantize_nv4(dev(w)), w)


def test_head_sized_int2_from_mx8(gpu, F):
    """The fast head's INT2 copy of a 248,320 x 2560 MXFP8 head straight from
    the packed rows equals quantize_int2 of the HIP fp32 dequant."""
    g = torch.Generator(device=gpu).manual_seed(3)
    w = torch.randn((248320, 2560), generator=g, device=gpu) * 0.02
    q, s = F.quantize_mx8(w)
    del w
    P, S = F.requantize_mx8(q, s, "int2", group=16)
    wf = F.mx8_dequant(q.view(torch.float8_e4m3fn), s)
    P2, S2 = F.quantize_int2(wf, group=16)
    assert torch.equal(P, P2) and torch.equal(S.view(torch.int16), S2.view(torch.int16))
    rows = torch.randperm(248320, generator=g, device=gpu)[:256].sort().values
    Po, So = oq.quantize_int2(wf[rows].cpu().numpy(), group=16)
    assert same(np_(P[rows]), Po) and same(np_(S[rows]), So)
    P, S, R = F.quantize_int2(wf, scale_fmt="e4m3", group=16)         # the row-scaled e4m3 form
    check("int2e", (P[rows], S[rows], R[rows]), wf[rows].cpu().numpy())
