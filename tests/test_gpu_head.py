"""GPU parity of the fast LM head (INT2 coarse -> top-C -> exact MXFP8 refine)
and of the draft head's pieces.

The oracle's coarse logits are the exact sums rounded to fp32 (the reference
accumulates in fp32 in an order its kernel leaves open); the GPU's coarse
sums run on MFMA and lie within oracle.ordered.mfma_bound of the exact sums,
so in bf16 they agree with the oracle's except for rare one-ulp flips, and
the selected set equals the oracle's except where such a flip decides
membership.  The selection is exact on the GPU's own coarse logits (bf16 for
the target head, fp32 for the draft head); the rescore uses IEEE fma steps in
an order the oracle replays, so refined logits agree bit for bit.  Full size:
V = 248,320, K = 2560, M = 3, G = 16, C = 512, N(0, 0.02) weights with 64
seeded rows x4, 32 seeded batches.
"""
import numpy as np
import pytest
import torch

from oracle import formats as fm
from oracle import gemv as og
from oracle import head as oh
from oracle import ordered
from oracle import quant as oq

from gpu_helpers import act, assert_tol, bf16_bits, bf16_dev, dev, to_f32, path_switch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def F():
    import fp4x_kernels
    return fp4x_kernels


def lpr_of(fmt, k):
    import _fp4x
    return _fp4x.layout(fmt, k)[0]


# ------------------------------------------------------------------ top-k
@pytest.mark.parametrize("V,C", [(248320, 512), (1000, 512), (4096, 2048), (50000, 2048), (100, 1), (5000, 2048),
                                 (65197, 64), (130000, 200), (262000, 100), (300000, 512), (600000, 64)])
def test_topk_rows_total_order(gpu, F, V, C):
    """Rows of 1, 2 and 4 slice vectors per thread, candidate counts for the
    rank sort (C <= about 200) and the bitonic sorts; row 2's specials widen its
    key range past 256 values (two radix rounds), rows 0-1 stay within it."""
    rng = np.random.default_rng(V + C)
    vals = fm.round_bf16((rng.standard_normal((3, V)) * 2).astype(np.float32))
    vals[1] = fm.round_bf16(np.round(vals[1] * 4) / 4)          # heavy ties
    bits = fm.bf16_bits(vals)
    bits[2, :7] = [0x8000, 0x0000, 0x7FC0, 0xFF80, 0x7F80, 0xFFC1, 0x0001]   # -0, +0, NaN, -inf, inf, -NaN, denormal
    t = dev(bits.view(np.int16)).view(torch.bfloat16)
    got = F.topk_rows(t, C).cpu().numpy()
    want = oh.topk_total_order(bits, C)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("V,C", [(65197, 64), (65197, 256), (248320, 512), (3000, 100), (20000, 2048),
                                 (600000, 64), (300000, 512)])
def test_topk_rows_fp32_total_order(gpu, F, V, C):
    """fp32 rows (the draft head selects on fp32 coarse logits): values that
    share a bf16 rounding but differ in fp32, exact fp32 ties, the specials."""
    rng = np.random.default_rng(V + 7 * C)
    vals = (rng.standard_normal((3, V)) * 2).astype(np.float32)
    vals[1] = fm.round_bf16(vals[1])                                  # bf16 ties ...
    vals[1, ::3] = np.nextafter(vals[1, ::3], np.float32(np.inf))     # ... split in fp32
    vals[1, ::7] = vals[1, 0]                                         # exact fp32 ties
    vals[2, :8] = [-0.0, 0.0, np.nan, -np.inf, np.inf, -np.nan, 1e-45, -1e-45]
    t = dev(vals)
    got = F.topk_rows(t, C).cpu().numpy()
    assert np.array_equal(got, oh.topk_total_order(vals, C))


def test_topk_rows_fp32_exact_and_tail_paths(gpu, F):
    """fp32: all-equal rows (the exact path, 32-bit radix rounds), a row whose
    winners sit in its last partial 16-byte item, and a strided view."""
    V, C = 300000, 512
    vals = np.full((2, V), 1.5, np.float32)
    vals[1, 123456] = 1.5000001
    got = F.topk_rows(dev(vals), C).cpu().numpy()
    assert np.array_equal(got, oh.topk_total_order(vals, C))
    assert got[0].tolist() == list(range(C)) and got[1, 0] == 123456
    rng = np.random.default_rng(3)
    V = 50003
    vals = rng.standard_normal((3, V)).astype(np.float32)
    vals[0, -3:] = [9.0, 8.5, 9.0]
    big = np.full((3, V + 5), np.inf, np.float32)
    big[:, :V] = vals
    t = dev(big)[:, :V]
    got = F.topk_rows(t, 64).cpu().numpy()
    assert np.array_equal(got, oh.topk_total_order(vals, 64))
    assert got[0, :3].tolist() == [V - 3, V - 1, V - 2]


@pytest.mark.parametrize("view", [False, True])
def test_topk_tail_item(gpu, F, view):
    """Rows of 50,003 elements whose largest values sit in the last, partial
    8-element item (read whole, the elements past V masked), from a padded copy
    and from a view whose stride already covers round_up(V, 8)."""
    rng = np.random.default_rng(50003)
    V, C = 50003, 64
    vals = fm.round_bf16(rng.standard_normal((3, V)).astype(np.float32))
    vals[0, -3:] = [9.0, 8.5, 9.0]                   # ties at the very end
    vals[1, -1] = 7.0
    bits = fm.bf16_bits(vals)
    if view:
        big = np.full((3, V + 5), 0x7F80, np.uint16)   # +inf past V: must not be selected
        big[:, :V] = bits
        t = dev(big.view(np.int16)).view(torch.bfloat16)[:, :V]
    else:
        t = dev(bits.view(np.int16)).view(torch.bfloat16)
    got = F.topk_rows(t, C).cpu().numpy()
    assert np.array_equal(got, oh.topk_total_order(bits, C))
    assert got[0, :3].tolist() == [V - 3, V - 1, V - 2] and got[1, 0] == V - 1


def test_topk_all_equal_exact_path(gpu, F):
    V, C = 300000, 512
    bits = np.full((2, V), fm.bf16_bits(np.float32(1.5)), np.uint16)
    bits[1, 123456] = fm.bf16_bits(np.array([2.0], np.float32))[0]
    t = dev(bits.view(np.int16)).view(torch.bfloat16)
    got = F.topk_rows(t, C).cpu().numpy()
    assert np.array_equal(got, oh.topk_total_order(bits, C))
    assert got[0].tolist() == list(range(C)) and got[1, 0] == 123456


def test_topk_rearms_across_calls_and_paths(gpu, F):
    """The shared workspace carries no state from one call to the next:
    alternating candidate-path and exact-path rows (and row counts) on one
    workspace keeps every result exact."""
    rng = np.random.default_rng(77)
    V, C = 248320, 512
    normal = fm.bf16_bits(fm.round_bf16(rng.standard_normal((3, V)).astype(np.float32)))
    ties = np.full((2, V), fm.bf16_bits(np.array([0.75], np.float32))[0], np.uint16)
    want_n = oh.topk_total_order(normal, C)
    want_t = oh.topk_total_order(ties, C)
    tn = dev(normal.view(np.int16)).view(torch.bfloat16)
    tt = dev(ties.view(np.int16)).view(torch.bfloat16)
    for _ in range(3):
        assert np.array_equal(F.topk_rows(tn, C).cpu().numpy(), want_n)
        assert np.array_equal(F.topk_rows(tt, C).cpu().numpy(), want_t)
        assert np.array_equal(F.topk_rows(tn[1:2], C).cpu().numpy(), want_n[1:2])


def test_topk_ignores_stale_workspace(gpu, F):
    """A row of 12,503 slices (not a multiple of the 8-slice padding): the
    workspace's padding entries, never written, hold 0xff from an earlier call
    and must not raise the threshold."""
    rng = np.random.default_rng(5)
    V, C = 200040, 512
    bits = fm.bf16_bits(fm.round_bf16(rng.standard_normal((2, V)).astype(np.float32)))
    t = dev(bits.view(np.int16)).view(torch.bfloat16)
    ws = F._topk_workspace(t.device, 16 << 20)
    ws.fill_(255)
    assert np.array_equal(F.topk_rows(t, C).cpu().numpy(), oh.topk_total_order(bits, C))


# ------------------------------------------------------------------ refine
def test_refine_mx8_exact(gpu, F):
    rng = np.random.default_rng(21)
    V, K, M, C = 20000, 2560, 3, 512
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    q, s = oq.quantize_mx8(w)
    x, xb = act(rng, M, K)
    idx = np.stack([rng.choice(V, C, replace=False) for _ in range(M)]).astype(np.int64)
    out = torch.zeros((M, V), dtype=torch.bfloat16, device=gpu)
    F.refine_mx8_(out, bf16_dev(x), dev(idx), dev(q), dev(s))
    exact = oh.mx8_rows(xb, q, s, idx, lpr_of(0, K))
    got = bf16_bits(out)
    assert np.array_equal(np.take_along_axis(got, idx, 1), fm.bf16_bits(exact))
    mask = np.ones((M, V), bool)
    np.put_along_axis(mask, idx, False, 1)
    assert np.all(got[mask] == 0)
    # fp32 out: the exact sums themselves
    out32 = torch.zeros((M, V), dtype=torch.float32, device=gpu)
    F.refine_mx8_(out32, bf16_dev(x), dev(idx), dev(q), dev(s))
    assert np.array_equal(np.take_along_axis(out32.cpu().numpy(), idx, 1).view(np.uint32), exact.view(np.uint32))
    ref = og.matmul_f32(x, oq.mx8_dequant(q[idx[0]], s[idx[0]]))[0]
    assert_tol(np.take_along_axis(out32.cpu().numpy(), idx, 1)[0], ref, what="refine vs matmul")


# ------------------------------------------------------------------ INT2 coarse
@pytest.mark.parametrize("M", [1, 3, 16])
def test_int2_logits_exact(gpu, F, M):
    rng = np.random.default_rng(31 + M)
    V, K = 8192, 2560
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    P, S = oq.quantize_int2(w)
    x, xb = act(rng, M, K)
    y = F.int2_logits(bf16_dev(x), dev(P), dev(S), V)             # fp32 out (reference default)
    exact = oh.int2_coarse(xb, P, S, 16)                          # the exact sums rounded to fp32
    wop = og.operand("int2", P, S)
    assert np.all(np.abs(y.cpu().numpy() - ordered.exact_sum(x, wop)) <= ordered.mfma_bound(x, wop))
    assert_tol(y.cpu().numpy(), og.int2_logits(x, P, S), what="int2 vs matmul")
    yb = F.int2_logits(bf16_dev(x), dev(P), dev(S), V, out_dtype=torch.bfloat16)
    eq = bf16_bits(yb) == fm.bf16_bits(exact)
    print(f"int2 M={M}: bf16 coarse equal to the rounded exact sums: {eq.mean():.6f}")
    assert eq.mean() >= 0.999


def test_int2_row_scale_variant(gpu, F):
    rng = np.random.default_rng(41)
    V, K = 2048, 2560
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    P, S, R = oq.quantize_int2(w, scale_fmt="e4m3")
    x, _ = act(rng, 3, K)
    y = F.int2_logits(bf16_dev(x), dev(P), dev(S).view(torch.float8_e4m3fn), V, RS=dev(R))
    assert_tol(y.cpu().numpy(), og.int2_logits(x, P, S, scale_fmt="e4m3", RS=R), what="int2 e4m3 + RS")


# ------------------------------------------------------------------ full head
def synth_head(gpu, F, V=248320, K=2560, seed=2):
    g = torch.Generator(device=gpu).manual_seed(seed)
    w = torch.randn((V, K), generator=g, device=gpu) * 0.02
    rows = torch.randperm(V, generator=g, device=gpu)[:64]
    w[rows] *= 4
    q, s = F.quantize_mx8(w)
    del w
    P, S = F.quantize_int2(F.mx8_dequant(q, s), group=16)
    return q, s, P, S


def test_fast_head_full_size_32_batches(gpu, F):
    """32 seeded M = 3 batches through the production path (int2_topk, then
    refine_mx8_), each row against the oracle's fast head: coarse values
    within the MFMA bound (plus half a bf16 ulp) of the exact sums; the
    selection exact on the GPU's own coarse logits; the selected set equal to
    the oracle's except where a flipped coarse value decides membership, and
    identical on at least 95% of the rows; refined logits bit-exact; the argmax equal to the oracle's on every row.
    Prints the set-identity rate and the argmax agreement with the exact
    full-vocabulary MXFP8 head."""
    V, K, M, C, B = 248320, 2560, 3, 512, 32
    q, s, P, S = synth_head(gpu, F, V, K)
    Pn, Sn, qn, sn = P.cpu().numpy(), S.cpu().numpy(), q.cpu().numpy(), s.cpu().numpy()
    xs = [act(np.random.default_rng(1000 + b), M, K) for b in range(B)]
    xall = np.concatenate([x for x, _ in xs])                       # [B * M, K]
    # GPU: the fast head's production calls, one batch at a time
    coarse_bits, sel, outs, full_am = [], [], [], []
    for x, _ in xs:
        xt = bf16_dev(x)
        coarse, idx = F.int2_topk(xt, P, S, V, C, sorted=False)
        coarse_bits.append(bf16_bits(coarse))
        sel.append(idx.cpu().numpy())
        outs.append(bf16_bits(F.refine_mx8_(coarse, xt, idx, q, s)))
        full_am.append(F.mx8_linear(xt, q, s, (32, 512, 1, 4), torch.float32).argmax(-1).cpu().numpy())
    coarse_bits, sel, outs = np.concatenate(coarse_bits), np.concatenate(sel), np.concatenate(outs)
    full_am = np.concatenate(full_am)
    # oracle coarse (exact sums rounded to fp32, then bf16) and the bound, one pass over the head
    xd = xall.astype(np.float64)
    o_coarse = np.empty((B * M, V), np.uint16)
    worst = 0.0
    for r0 in range(0, V, 16384):
        r1 = min(V, r0 + 16384)
        w = fm.bf16_to_f32(ordered.int2_operand_bits(Pn[r0:r1], Sn[r0:r1], 16)).astype(np.float64)
        ex = xd @ w.T
        bound = (3 * (K // 32) + 17) * 2.0 ** -23 * (np.abs(xd) @ np.abs(w).T)
        o_coarse[:, r0:r1] = fm.bf16_bits(ex.astype(np.float32))
        cf = fm.bf16_to_f32(coarse_bits[:, r0:r1]).astype(np.float64)
        lim = bound + np.abs(cf) * 2.0 ** -8
        assert np.all(np.abs(cf - ex) <= lim), f"coarse rows {r0}..{r1}"
        worst = max(worst, float((np.abs(cf - ex) / lim).max()))
        del w, ex, bound, cf, lim
    diff = coarse_bits != o_coarse
    print(f"coarse bf16 flips against the rounded exact sums: {int(diff.sum())} of {diff.size} "
          f"(max |d| / bound {worst:.3g})")
    assert diff.mean() <= 1e-3
    # selection (the set, in index order): exact on the GPU's coarse; the
    # oracle's set up to flipped entries
    assert np.array_equal(sel, np.sort(oh.topk_total_order(coarse_bits, C), 1))
    o_idx = oh.topk_total_order(o_coarse, C)
    same_set = 0
    for r in range(B * M):
        sym = set(sel[r].tolist()) ^ set(o_idx[r].tolist())
        assert all(diff[r, i] for i in sym), f"row {r}: set differs beyond flipped entries"
        same_set += not sym
    # and a floor on identity itself: a flip at the boundary is a rare event, so
    # a drift that flips many boundary entries fails here even if each is a flip
    assert same_set >= 0.95 * B * M, f"top-{C} set identical to the oracle's on only {same_set} of {B * M} rows"
    # refined logits: the rescore of the selected rows, bit for bit
    xb = fm.bf16_bits(xall)
    exact = oh.mx8_rows(xb, qn, sn, sel, lpr_of(0, K))
    assert np.array_equal(np.take_along_axis(outs, sel, 1), fm.bf16_bits(exact)), "refined logits"
    # the oracle's fast head output and its argmax
    o_exact = oh.mx8_rows(xb, qn, sn, o_idx, lpr_of(0, K))
    o_out = o_coarse.copy()
    np.put_along_axis(o_out, o_idx, fm.bf16_bits(o_exact), 1)
    am = np.argmax(fm.bf16_to_f32(outs), -1)
    assert np.array_equal(am, np.argmax(fm.bf16_to_f32(o_out), -1))
    print(f"fast head, {B * M} rows: top-{C} set identical to the oracle's on {same_set}; argmax equal to the "
          f"oracle's on all; argmax equal to the exact MXFP8 head on {int((am == full_am).sum())}")


# ------------------------------------------------------------------ INT2 streaming kernel
@pytest.mark.parametrize("M,rs,one,K,e4m3", [(3, False, 0, 2560, False), (16, False, 0, 2560, False),
                                              (3, True, 0, 2560, False), (3, False, 1, 2560, False),
                                              (3, False, 2, 2560, False), (3, False, 0, 1536, False),
                                              (3, True, 0, 2560, True), (16, True, 1, 2560, True),
                                              (3, True, 2, 1536, True)])
def test_int2_stream(gpu, F, M, rs, one, K, e4m3, monkeypatch):
    """Heads of at least one tile per two waves of the grid take the streaming
    kernel (16 waves per CU, LDS ring of direct loads); N tail of 40 rows.
    one = 1: just under one tile per wave (the 65,197-row draft subset on 256
    CUs: some workgroups have a wave with no tile), 3 rows past the last full
    tile; one = 2: 10 tiles per CU (six waves of a workgroup without a tile),
    5 rows past the last full tile; K = 1536: three units per tile instead of
    five.  e4m3: the row-scaled form (e4m3 group scales, the quantizer's fp32
    row scales as rs)."""
    _int2_stream_case(F, M, rs, one, K, e4m3, 16, monkeypatch)


@pytest.mark.parametrize("M,rs,one,K", [(3, False, 0, 2560), (16, True, 1, 2560), (3, False, 2, 1536)])
def test_int2_stream_g32(gpu, F, M, rs, one, K, monkeypatch):
    """fp16 group scales at G = 32 (the plugin's FP4X_HEAD_G=32) stream as
    e4m3 ones do: 32 scale bytes per row and unit, two fp16 scales per 64-weight
    chunk; the same checks."""
    _int2_stream_case(F, M, rs, one, K, False, 32, monkeypatch)


def _int2_stream_case(F, M, rs, one, K, e4m3, G, monkeypatch):
    rng = np.random.default_rng(77 + M + rs + 5 * one + K + 3 * e4m3 + G)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    V = {0: 4 * 8 * 16 * cus + 40, 1: 16 * (16 * cus - 21) - 3, 2: 16 * 10 * cus - 5}[one]
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    if e4m3:
        P, S, R = oq.quantize_int2(w, scale_fmt="e4m3", group=16)
        Sd = dev(S).view(torch.float8_e4m3fn)
    else:
        P, S = oq.quantize_int2(w, group=G)
        R = (rng.random(V) + 0.5).astype(np.float32) if rs else None
        Sd = dev(S)
    del w
    print(f"int2 stream V={V} K={K} M={M} rs={rs} e4m3={e4m3} G={G}", flush=True)
    x, xb = act(rng, M, K)
    args = (bf16_dev(x), dev(P), Sd, V)
    kw = {"RS": dev(R)} if rs else {}
    y = F.int2_logits(*args, **kw).cpu().numpy()
    with path_switch(monkeypatch, "FP4X_INT2_STREAM"):
        y_core = F.int2_logits(*args, **kw).cpu().numpy()
    assert not np.array_equal(y.view(np.uint32), y_core.view(np.uint32)), "streaming kernel not taken"
    worst = 0.0
    for r0 in range(0, V, 16384):
        r1 = min(V, r0 + 16384)
        wop = og.operand("int2", P[r0:r1], S[r0:r1], **({"scale_fmt": "e4m3"} if e4m3 else {}))
        exact = ordered.exact_sum(x, wop)
        bound = ordered.mfma_bound(x, wop)
        if rs:
            exact = exact * R[r0:r1]
            bound = bound * R[r0:r1] * (1 + 2.0 ** -23) + np.abs(exact) * 2.0 ** -23
        for got in (y[:, r0:r1], y_core[:, r0:r1]):
            assert np.all(np.abs(got - exact) <= bound), float((np.abs(got - exact) / bound).max())
        worst = max(worst, float((np.abs(y[:, r0:r1] - exact) / bound).max()))
    print(f"int2 stream V={V} M={M} rs={rs} e4m3={e4m3} G={G}: max |y - exact| / bound = {worst:.3g}")
    # bf16 logits round the same sums
    yb = F.int2_logits(*args, out_dtype=torch.bfloat16, **kw)
    assert np.array_equal(bf16_bits(yb), fm.bf16_bits(y))


# ------------------------------------------------------------------ fused coarse + top-k
@pytest.mark.parametrize("V,M,rs,C,f32", [(248320, 3, False, 512, False), (248320, 16, False, 512, False),
                                          (200040, 3, True, 512, False), (50000, 3, False, 512, False),
                                          (65197, 3, False, 64, False), (20000, 3, False, 64, False),
                                          (65197, 3, False, 64, True), (248320, 3, False, 512, True),
                                          (20000, 16, False, 256, True), (248320, 3, "e4m3", 512, False),
                                          (65197, 3, "e4m3", 64, True), (248320, 3, "g32", 1024, False)])
def test_int2_topk_fused_equals_separate(gpu, F, V, M, rs, C, f32):
    """int2_topk (slice maxima from the streaming coarse kernel's epilogue where
    it streams, else a slice-max launch) equals int2_logits + topk_rows bit for
    bit, and its selection is the oracle's total order on its own logits; for
    fp16 (G = 16 and 32) and for e4m3 (row-scaled) group scales."""
    K = 2560
    g = torch.Generator(device=gpu).manual_seed(V + M)
    w = torch.randn((V, K), generator=g, device=gpu) * 0.02
    w[torch.randperm(V, generator=g, device=gpu)[:64]] *= 4
    if rs == "e4m3":                                  # the row-scaled form: its own row scales as RS
        P, S, R = F.quantize_int2(w, scale_fmt="e4m3", group=16)
    elif rs == "g32":                                 # fp16 scales per 32 (FP4X_HEAD_G=32, C = 1024)
        P, S = F.quantize_int2(w, group=32)
        R = None
    else:
        P, S = F.quantize_int2(w, group=16)
        R = (torch.rand(V, generator=g, device=gpu) + 0.5) if rs else None
    del w
    rng = np.random.default_rng(V + M)
    x, _ = act(rng, M, K)
    xt = bf16_dev(x)
    dt = torch.float32 if f32 else torch.bfloat16
    coarse, idx = F.int2_topk(xt, P, S, V, C, RS=R, out_dtype=dt)
    coarse2 = F.int2_logits(xt, P, S, V, RS=R, out_dtype=dt)
    idx2 = F.topk_rows(coarse2, C)
    assert torch.equal(coarse.view(torch.int16 if not f32 else torch.int32),
                       coarse2.view(torch.int16 if not f32 else torch.int32))
    assert torch.equal(idx, idx2)
    host = coarse.cpu().numpy() if f32 else bf16_bits(coarse)
    assert np.array_equal(idx.cpu().numpy(), oh.topk_total_order(host, C))
    # sorted=False (the heads scatter at the indices): the same set per row (in
    # increasing index order for bf16 logits, with up to 1024 candidates, as a
    # top-512 leaves, or more, as a top-1024 has; the sorted order for fp32
    # ones)
    coarse3, idx3 = F.int2_topk(xt, P, S, V, C, RS=R, out_dtype=dt, sorted=False)
    assert torch.equal(coarse3.view(torch.int16 if not f32 else torch.int32),
                       coarse.view(torch.int16 if not f32 else torch.int32))
    if f32:
        assert torch.equal(idx3, idx)
    else:
        assert torch.equal(idx3, torch.sort(idx, dim=1).values)


@pytest.mark.parametrize("case,V,C", [("short_row", 3000, 512), ("all_tied", 50000, 512), ("wide_tie", 248320, 512),
                                      ("top1024", 248320, 1024), ("tie1024", 248320, 1024)])
def test_int2_topk_set_only_paths(gpu, F, case, V, C):
    """sorted=False on the selection's other paths: a row of at most 4096
    elements (sorted whole), every row element tied (the exact threshold
    path), 2000 identical rows holding the top 512 (more candidates at the
    threshold than the candidate buffers take), a top-1024 (more candidates
    than the workgroup's threads: four per thread) and a top-1024 whose last
    places are 1500 tied rows.  The set equals the sorted call's, which is the
    oracle's total order on the same logits; the top-1024 sets come out in
    increasing index order."""
    K, M = 2560, 3
    g = torch.Generator(device=gpu).manual_seed(V + C)
    w = torch.randn((V, K), generator=g, device=gpu) * 0.02
    if case == "all_tied":
        w[:] = w[0]
    elif case == "wide_tie":
        w[torch.randperm(V, generator=g, device=gpu)[:2000]] = w[0] * 4
    elif case == "tie1024":
        sel = torch.randperm(V, generator=g, device=gpu)
        w[sel[:600]] *= 8
        w[sel[600:2100]] = w[sel[600]] * 4
    P, S = F.quantize_int2(w, group=16)
    del w
    xt = bf16_dev(act(np.random.default_rng(V), M, K)[0])
    coarse, idx = F.int2_topk(xt, P, S, V, C)
    coarse3, idx3 = F.int2_topk(xt, P, S, V, C, sorted=False)
    assert torch.equal(coarse.view(torch.int16), coarse3.view(torch.int16))
    assert np.array_equal(idx.cpu().numpy(), oh.topk_total_order(bf16_bits(coarse), C))
    assert torch.equal(torch.sort(idx3, dim=1).values, torch.sort(idx, dim=1).values)
    if case == "all_tied":
        assert torch.equal(torch.sort(idx3, dim=1).values, torch.arange(C, device=gpu).expand(M, C))
    if C > 512:
        assert torch.equal(idx3, torch.sort(idx3, dim=1).values)


# ------------------------------------------------------------------ draft head (NVFP4 rescore)
def test_refine_nv4_exact(gpu, F):
    """refine_nv4: the rescore kernel's fma order replayed by the oracle, bit for
    bit, times gs; NaN for candidates outside [0, V); within tolerance of the
    fp32 matmul of the dequantized rows."""
    import _fp4x
    rng = np.random.default_rng(31)
    V, K, M, C = 20000, 2560, 3, 64
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    P, S, gs = oq.quantize_nv4(w)
    x, xb = act(rng, M, K)
    idx = np.stack([rng.choice(V, C, replace=False) for _ in range(M)]).astype(np.int64)
    out = F.refine_nv4(bf16_dev(x), dev(idx), dev(P), dev(S).view(torch.float8_e4m3fn), gs)
    exact = oh.nv4_rows(xb, P, S, gs, idx, lpr_of(_fp4x.FMT_NV4, K))
    assert out.shape == (M, C) and out.dtype == torch.float32
    assert np.array_equal(out.cpu().numpy().view(np.uint32), exact.view(np.uint32))
    ref = og.matmul_f32(x[:1], oq.dequant_nv4_operand(P[idx[0]], S[idx[0]]))[0] * np.float32(gs)
    assert_tol(out.cpu().numpy()[0], ref, what="refine_nv4 vs matmul")
    bad = idx.copy()
    bad[1, 5], bad[2, 0] = -1, V
    out2 = F.refine_nv4(bf16_dev(x), dev(bad), dev(P), dev(S).view(torch.float8_e4m3fn), gs).cpu().numpy()
    assert np.isnan(out2[1, 5]) and np.isnan(out2[2, 0])
    keep = ~np.isnan(out2)
    assert np.array_equal(out2[keep].view(np.uint32), exact[keep].view(np.uint32))


@pytest.mark.parametrize("dc", [64, 0])
def test_draft_head(gpu, F, dc):
    """The plugin's draft head over a vocabulary subset (x/fp4patch.py:309-330):
    -inf outside the subset; with dc > 0 the top dc of the GPU's own fp32
    INT2 coarse logits (the oracle's total order) carry their exact NVFP4
    logits, and those coarse logits lie within the MFMA bound of the exact
    sums; with dc = 0 the subset carries the NVFP4 GEMV."""
    import _fp4x
    import fp4patch
    rng = np.random.default_rng(32 + dc)
    vocab, K, M, nsub = 30000, 2560, 3, 6000
    w = (rng.standard_normal((vocab, K)) * 0.02).astype(np.float32)
    P, S, gs = oq.quantize_nv4(w)
    ids_np = np.sort(rng.choice(vocab, nsub, replace=False)).astype(np.int64)
    x, xb = act(rng, M, K)
    h = bf16_dev(x)
    st = fp4patch._draft_prepare(F, dev(P), dev(S).view(torch.float8_e4m3fn), gs, dev(ids_np), dc)
    full = fp4patch._draft_logits(F, h, st, vocab, dc)
    got = bf16_bits(full)
    outside = np.ones((M, vocab), bool)
    if dc:
        co = F.int2_logits(h, *st["c"], nsub).cpu().numpy()         # fp32, as x/fp4patch.py:313
        P2, S2 = (t.cpu().numpy() for t in st["c"])
        wop = og.operand("int2", P2, S2)
        assert np.all(np.abs(co - ordered.exact_sum(x, wop)) <= ordered.mfma_bound(x, wop))
        cand = oh.topk_total_order(co, dc)
        vals = oh.nv4_rows(xb, P[ids_np], S[ids_np], gs, cand, lpr_of(_fp4x.FMT_NV4, K))
        pos = ids_np[cand]
        assert np.array_equal(np.take_along_axis(got, pos, 1), fm.bf16_bits(vals))
        np.put_along_axis(outside, pos, False, 1)
    else:
        sub = og.matmul_f32(x, oq.dequant_nv4_operand(P[ids_np], S[ids_np])) * np.float32(gs)
        assert_tol(to_f32(full)[:, ids_np], sub, what="draft subset GEMV")
        outside[:, ids_np] = False
    assert np.all(got[outside] == 0xFF80)


@pytest.mark.parametrize("vocab", [248320, 30001, 300])
def test_scatter_draft(gpu, F, vocab):
    """The draft logits scatter equals torch.full(-inf) + scatter_ of
    bf16(vals * inv_t) bit for bit (x/fp4patch.py:316-320), on 16-byte rows and
    on odd row lengths (unaligned rows, ragged tails); out-of-range cand or ids
    entries leave -inf."""
    g = torch.Generator(device=gpu).manual_seed(vocab)
    M, C = 3, 64
    nsub = min(vocab, 6000)
    ids = torch.sort(torch.randperm(vocab, generator=g, device=gpu)[:nsub]).values
    cand = torch.stack([torch.randperm(nsub, generator=g, device=gpu)[:C] for _ in range(M)])
    vals = torch.randn((M, C), generator=g, device=gpu) * 8
    for inv_t in (None, torch.full((1,), 1.0 / 0.7, device=gpu)):
        got = F.scatter_draft(vals, cand, ids, vocab, inv_t)
        v = vals if inv_t is None else vals * inv_t
        ref = torch.full((M, vocab), float("-inf"), dtype=torch.bfloat16, device=gpu)
        ref.scatter_(1, ids[cand], v.to(torch.bfloat16))
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    bad = cand.clone()
    bad[0, 0], bad[1, 1] = -1, nsub                  # out of range: not written
    got = F.scatter_draft(vals, bad, ids, vocab)
    ref = torch.full((M, vocab), float("-inf"), dtype=torch.bfloat16, device=gpu)
    keep = torch.ones_like(cand, dtype=torch.bool)
    keep[0, 0] = keep[1, 1] = False
    for m in range(M):
        ref[m, ids[cand[m][keep[m]]]] = vals[m][keep[m]].to(torch.bfloat16)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("vocab,C,dense", [(248320, 64, False), (30001, 300, False), (30001, 600, True), (300, 64, True)])
def test_draft_nv4_fused(gpu, F, vocab, C, dense):
    """draft_nv4 (the rescore and the scatter in one launch) equals refine_nv4
    followed by scatter_draft bit for bit: with and without inv_t, on 16-byte
    and odd row lengths, with more candidates than threads, with many
    candidates in one 2048-column block (dense ids: the fill skips many
    columns of each 8-column store), with repeated candidates, and with
    out-of-range cand entries left -inf."""
    g = torch.Generator(device=gpu).manual_seed(vocab + C)
    M, K = 3, 2560
    nsub = min(vocab, 6000)
    ids = torch.arange(nsub, device=gpu) if dense else \
        torch.sort(torch.randperm(vocab, generator=g, device=gpu)[:nsub]).values
    P, S, gs = F.quantize_nv4(torch.randn((nsub, K), generator=g, device=gpu) * 0.02)
    h = (torch.randn((M, K), generator=g, device=gpu)).to(torch.bfloat16)
    cand = torch.stack([torch.randperm(nsub, generator=g, device=gpu)[:C] for _ in range(M)])
    cand[2, 1] = cand[2, 0]                           # a repeated candidate
    bad = cand.clone()
    bad[0, 0], bad[1, C - 1] = -1, nsub               # out of range: not written
    for cc in (cand, bad):
        for inv_t in (None, torch.full((1,), 1.0 / 0.7, device=gpu)):
            print(f"vocab={vocab} C={C} dense={dense} inv_t={inv_t is not None}", flush=True)
            got = F.draft_nv4(h, cc, P, S, gs, ids, vocab, inv_t)
            ref = F.scatter_draft(F.refine_nv4(h, cc, P, S, gs), cc, ids, vocab, inv_t)
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
            assert int((got.view(torch.int16) != -128).sum()) == len(set(
                (m, int(i)) for m in range(M) for i in cc[m].tolist() if 0 <= i < nsub))
