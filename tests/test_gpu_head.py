"""GPU parity of the fast LM head (INT2 coarse -> top-C -> exact MXFP8 refine).

The oracle replays the kernels' summation order.  The rescore uses IEEE fma
steps, so refined logits and the argmax agree bit for bit; the top-C
selection is exact on given coarse logits; the coarse INT2 sums run on MFMA,
whose internal rounding the oracle bounds (oracle.ordered.mfma_bound) rather
than replays, so coarse logits agree bit for bit in bf16 except for rare
one-ulp flips, and the selected set equals the oracle's up to those flips.  Full size: V = 248,320, K = 2560, M = 3, G = 16,
C = 512, N(0, 0.02) weights with 64 seeded rows x4.
"""
import numpy as np
import pytest
import torch

from oracle import formats as fm
from oracle import gemv as og
from oracle import head as oh
from oracle import ordered
from oracle import quant as oq

from gpu_helpers import act, assert_tol, bf16_bits, bf16_dev, dev, to_f32

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
    exact = oh.int2_coarse(xb, P, S, 16, lpr_of(5, K))
    from oracle import ordered
    wop = og.operand("int2", P, S)
    bound = ordered.mfma_bound(x, wop) + ordered.step_bound(x, wop, 64, lpr_of(5, K))
    assert np.all(np.abs(y.cpu().numpy() - ordered.exact_sum(x, wop)) <= ordered.mfma_bound(x, wop))
    assert np.all(np.abs(y.cpu().numpy() - exact) <= bound)
    assert_tol(y.cpu().numpy(), og.int2_logits(x, P, S), what="int2 vs matmul")
    yb = F.int2_logits(bf16_dev(x), dev(P), dev(S), V, out_dtype=torch.bfloat16)
    eq = bf16_bits(yb) == fm.bf16_bits(exact)
    print(f"int2 M={M}: bf16 coarse equal to the ordered replay: {eq.mean():.6f}")
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


def test_fast_head_full_size_exact(gpu, F):
    V, K, M, C = 248320, 2560, 3, 512
    q, s, P, S = synth_head(gpu, F, V, K)
    rng = np.random.default_rng(1000)
    x, xb = act(rng, M, K)
    xt = bf16_dev(x)
    coarse = F.int2_logits(xt, P, S, V, out_dtype=torch.bfloat16)
    idx = F.topk_rows(coarse, C)
    coarse_bits = bf16_bits(coarse)
    out = F.refine_mx8_(coarse, xt, idx, q, s)
    Pn, Sn, qn, sn = P.cpu().numpy(), S.cpu().numpy(), q.cpu().numpy(), s.cpu().numpy()
    o_coarse, o_idx, o_out = oh.fast_head(xb, Pn, Sn, 16, qn, sn, C, lpr_of(5, K), lpr_of(0, K))
    diff = coarse_bits != o_coarse
    print(f"fast head: coarse bf16 differing from the ordered replay: {int(diff.sum())} of {diff.size}")
    assert diff.mean() <= 1e-3
    # every coarse value (MFMA-accumulated, then rounded to bf16) lies within
    # the accumulation bound plus half a bf16 ulp of the exact sum
    w_op = fm.bf16_to_f32(ordered.int2_operand_bits(Pn, Sn, 16))
    xf = fm.bf16_to_f32(xb)
    exact_c = ordered.exact_sum(xf, w_op)
    cf = fm.bf16_to_f32(coarse_bits).astype(np.float64)
    bound = ordered.mfma_bound(xf, w_op) + np.abs(cf) * 2.0 ** -8
    assert np.all(np.abs(cf - exact_c) <= bound), float((np.abs(cf - exact_c) / bound).max())
    del w_op, exact_c, bound
    sel = idx.cpu().numpy()
    # selection is exact on the kernel's own coarse logits ...
    assert np.array_equal(sel, oh.topk_total_order(coarse_bits, C))
    # ... and the set equals the oracle's except where a flipped coarse value decides membership
    for m in range(M):
        sym = set(sel[m].tolist()) ^ set(o_idx[m].tolist())
        assert all(diff[m, i] for i in sym) or not sym, f"row {m}: set differs beyond flipped entries"
    # refined logits: exact rescore of the selected rows
    exact = oh.mx8_rows(xb, qn, sn, sel, lpr_of(0, K))
    got = bf16_bits(out)
    assert np.array_equal(np.take_along_axis(got, sel, 1), fm.bf16_bits(exact)), "refined logits"
    am = out.float().argmax(-1).cpu().numpy()
    assert np.array_equal(am, np.argmax(fm.bf16_to_f32(o_out), -1))
    # the exact full-vocabulary MXFP8 argmax agrees (true argmax inside the top-512)
    full = F.mx8_linear(xt, q, s, (32, 512, 1, 4), torch.float32)
    assert np.array_equal(am, full.argmax(-1).cpu().numpy())


# ------------------------------------------------------------------ INT2 streaming kernel
@pytest.mark.parametrize("M,rs,one", [(3, False, False), (16, False, False), (3, True, False), (3, False, True)])
def test_int2_stream(gpu, F, M, rs, one, monkeypatch):
    """Heads of at least 2 tiles per wave of the grid take the streaming kernel
    (one wave per tile, LDS ring of direct loads); N tail of 40 rows.  one:
    between 1 and 2 tiles per wave at 8 waves per CU (the 65,197-row draft
    subset on 256 CUs), 3 rows past the last full tile."""
    rng = np.random.default_rng(77 + M + rs + 5 * one)
    K = 2560
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    V = 16 * (16 * cus - 21) - 3 if one else 4 * 8 * 16 * cus + 40
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    P, S = oq.quantize_int2(w, group=16)
    del w
    R = (rng.random(V) + 0.5).astype(np.float32) if rs else None
    x, xb = act(rng, M, K)
    args = (bf16_dev(x), dev(P), dev(S), V)
    kw = {"RS": dev(R)} if rs else {}
    y = F.int2_logits(*args, **kw).cpu().numpy()
    monkeypatch.setenv("FP4X_INT2_STREAM", "0")
    y_core = F.int2_logits(*args, **kw).cpu().numpy()
    monkeypatch.delenv("FP4X_INT2_STREAM")
    assert not np.array_equal(y.view(np.uint32), y_core.view(np.uint32)), "streaming kernel not taken"
    worst = 0.0
    for r0 in range(0, V, 16384):
        r1 = min(V, r0 + 16384)
        wop = og.operand("int2", P[r0:r1], S[r0:r1])
        exact = ordered.exact_sum(x, wop)
        bound = ordered.mfma_bound(x, wop)
        if rs:
            exact = exact * R[r0:r1]
            bound = bound * R[r0:r1] * (1 + 2.0 ** -23) + np.abs(exact) * 2.0 ** -23
        for got in (y[:, r0:r1], y_core[:, r0:r1]):
            assert np.all(np.abs(got - exact) <= bound), float((np.abs(got - exact) / bound).max())
        worst = max(worst, float((np.abs(y[:, r0:r1] - exact) / bound).max()))
    print(f"int2 stream V={V} M={M} rs={rs}: max |y - exact| / bound = {worst:.3g}")
    # bf16 logits round the same sums
    yb = F.int2_logits(*args, out_dtype=torch.bfloat16, **kw)
    assert np.array_equal(bf16_bits(yb), fm.bf16_bits(y))


# ------------------------------------------------------------------ fused coarse + top-k
@pytest.mark.parametrize("V,M,rs,C", [(248320, 3, False, 512), (248320, 16, False, 512), (200040, 3, True, 512),
                                      (50000, 3, False, 512), (65197, 3, False, 64), (20000, 3, False, 64)])
def test_int2_topk_fused_equals_separate(gpu, F, V, M, rs, C):
    """int2_topk (slice maxima from the streaming coarse kernel's epilogue where
    it streams, else a slice-max launch) equals int2_logits + topk_rows bit for
    bit, and its selection is the oracle's total order on its own logits."""
    K = 2560
    g = torch.Generator(device=gpu).manual_seed(V + M)
    w = torch.randn((V, K), generator=g, device=gpu) * 0.02
    w[torch.randperm(V, generator=g, device=gpu)[:64]] *= 4
    P, S = F.quantize_int2(w, group=16)
    del w
    R = (torch.rand(V, generator=g, device=gpu) + 0.5) if rs else None
    rng = np.random.default_rng(V + M)
    x, _ = act(rng, M, K)
    xt = bf16_dev(x)
    coarse, idx = F.int2_topk(xt, P, S, V, C, RS=R)
    coarse2 = F.int2_logits(xt, P, S, V, RS=R, out_dtype=torch.bfloat16)
    idx2 = F.topk_rows(coarse2, C)
    assert np.array_equal(bf16_bits(coarse), bf16_bits(coarse2))
    assert torch.equal(idx, idx2)
    assert np.array_equal(idx.cpu().numpy(), oh.topk_total_order(bf16_bits(coarse), C))


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
    -inf outside the subset; with dc > 0 the top dc of the GPU's own INT2
    coarse logits (the oracle's total order) carry their exact NVFP4 logits;
    with dc = 0 the subset carries the NVFP4 GEMV."""
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
        co = F.int2_logits(h, *st["c"], nsub, out_dtype=torch.bfloat16)
        cand = oh.topk_total_order(bf16_bits(co), dc)
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
