"""GPU parity of the dense decode GEMVs against the oracle.

* dequant: the bf16 operand each kernel decodes is bit-exact with the
  oracle's dequantize-then-round (all formats, all fp8 codes).
* GEMV: |y - y_oracle| <= 1e-2 + 2e-3 |y_oracle| against the fp32-accumulated
  oracle, for M = 1..20 (M > 16 runs as 16-row launches), split-K and tails;
  and, in fp32, within the MFMA accumulation bound of the exact (float64)
  sum (oracle.ordered.mfma_bound).
"""
import numpy as np
import pytest
import torch

from oracle import formats as fm
from oracle import gemv as og
from oracle import ordered
from oracle import quant as oq

from gpu_helpers import act, assert_tol, bf16_bits, bf16_dev, dev, to_f32, path_switch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def F():
    import fp4x_kernels
    return fp4x_kernels


def weights(rng, n, k, scale=0.02):
    return (rng.standard_normal((n, k)) * scale).astype(np.float32)


# ------------------------------------------------------------------ dequant
def test_dequant_mx8_all_codes(gpu, F):
    """Every fp8 code under every e8m0 exponent 0..255 (row r uses exponent
    r): the bf16 operand of the GEMVs and the fp32 mx8_dequant are bit-exact
    with the oracle, including results that are bf16 or fp32 subnormals,
    zeros from underflow, and overflow to inf (exponent 255, 2^128 in fp32,
    as exp2 gives it); 0 x 2^128 is NaN, as in the reference's fp32 product."""
    codes = np.tile(np.arange(256, dtype=np.uint8), (256, 1))
    codes[codes == 0x7F] = 0x7E                      # the two NaN codes are checked below
    codes[codes == 0xFF] = 0xFE
    exps = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 8, 1)
    w, s = dev(codes), dev(exps)
    want32 = oq.mx8_dequant(codes, exps)
    got32 = F.mx8_dequant(w, s).cpu().numpy()
    nan = np.isnan(want32)
    assert np.array_equal(np.isnan(got32), nan)
    assert np.array_equal(got32[~nan].view(np.uint32), want32[~nan].view(np.uint32))
    got = bf16_bits(F.dequant_operand("mx8", w, None, s, K=256))
    want = fm.bf16_bits(want32)
    gnan = (got & 0x7FFF) > 0x7F80
    assert np.array_equal(gnan, nan)
    bad = (got != want) & ~nan
    assert not bad.any(), (f"{int(bad.sum())} operands differ, e.g. code {int(np.argwhere(bad)[0][1])} exponent "
                           f"{int(np.argwhere(bad)[0][0])}: {got[bad][0]:#06x} vs {want[bad][0]:#06x}")
    # NaN codes stay NaN under every finite scale
    nc = np.tile(np.array([0x7F, 0xFF] * 16, np.uint8), (255, 1))
    ne = np.arange(255, dtype=np.uint8)[:, None]
    gn = bf16_bits(F.dequant_operand("mx8", dev(nc), None, dev(ne), K=32))
    assert np.all((gn & 0x7FFF) > 0x7F80)


@pytest.mark.parametrize("fmt", ["w8", "w8_f16", "w6", "nv4", "int2", "int2_g32", "int2_g128", "int2_e4m3"])
def test_dequant_operand_bit_exact(gpu, F, fmt):
    rng = np.random.default_rng(1)
    n, k = 64, 512
    w = weights(rng, n, k)
    w[3] = 0.0
    if fmt.startswith("w8"):
        q, s = oq.quantize_w8(w)
        s16 = fmt == "w8_f16"
        sd = s.astype(np.float16) if s16 else s
        got = F.dequant_operand(fmt, dev(q), None, dev(sd), K=k)
        want = og.operand("w8", q, sd.astype(np.float32))
    elif fmt == "w6":
        L, H, S = oq.quantize_w6(w)
        got = F.dequant_operand("w6", dev(L), dev(H), dev(S), K=k)
        want = og.operand("w6", L, H, S)
    elif fmt == "nv4":
        P, S, gs = oq.quantize_nv4(w)
        got = F.dequant_operand("nv4", dev(P), None, dev(S), K=k)
        want = og.operand("nv4", P, S)
    elif fmt == "int2_e4m3":
        P, S, R = oq.quantize_int2(w, scale_fmt="e4m3")
        got = F.dequant_operand("int2_e4m3", dev(P), None, dev(S), K=k, G=16)
        want = og.operand("int2", P, S, scale_fmt="e4m3")
    else:
        G = {"int2": 16, "int2_g32": 32, "int2_g128": 128}[fmt]
        P, S = oq.quantize_int2(w, group=G)
        got = F.dequant_operand("int2", dev(P), None, dev(S), K=k, G=G)
        want = og.operand("int2", P, S)
    assert np.array_equal(bf16_bits(got), fm.bf16_bits(want))


# ------------------------------------------------------------------ GEMVs
def prep(fmt, rng, n, k):
    w = weights(rng, n, k)
    if fmt == "mx8":
        q, s = oq.quantize_mx8(w)
        return (dev(q), dev(s)), og.operand("mx8", q, s), 1.0
    if fmt == "w8":
        q, s = oq.quantize_w8(w)
        return (dev(q), dev(s)), og.operand("w8", q, s), 1.0
    if fmt == "w6":
        L, H, S = oq.quantize_w6(w)
        return (dev(L), dev(H), dev(S)), og.operand("w6", L, H, S), 1.0
    if fmt == "nv4":
        P, S, gs = oq.quantize_nv4(w)
        return (dev(P), dev(S).view(torch.float8_e4m3fn), gs), og.operand("nv4", P, S), gs
    if fmt == "bf16":
        wb = fm.round_bf16(w)
        return (bf16_dev(wb),), wb, 1.0
    raise ValueError(fmt)


def run(F, fmt, x_t, planes, ks, out_dtype=torch.bfloat16):
    if fmt == "mx8":
        return F.mx8_linear(x_t, *planes, (32, 64, ks, 4), out_dtype)
    if fmt == "w8":
        return F.w8_linear(x_t, *planes, (32, 64, ks, 4), out_dtype)
    if fmt == "w6":
        return F.w6_linear(x_t, *planes, (32, 64, ks, 4), out_dtype)
    if fmt == "nv4":
        return F.nv4_linear(x_t, *planes, (32, 64, 4, ks), out_dtype)
    return F.bf16_linear(x_t, *planes, (32, 64, ks, 4), out_dtype)


KPC = {"mx8": 16, "w8": 16, "w6": 32, "nv4": 32, "bf16": 16}
FMT = {"mx8": 0, "w8": 1, "w6": 3, "nv4": 4, "bf16": 7}


@pytest.mark.parametrize("fmt", ["mx8", "w8", "w6", "nv4", "bf16"])
@pytest.mark.parametrize("M", [1, 3, 5, 16, 20])
def test_gemv_parity(gpu, F, fmt, M):
    rng = np.random.default_rng(100 + M)
    n, k = 1000, 2560           # N tail: 1000 is not a multiple of any row tile
    planes, w_op, gs = prep(fmt, rng, n, k)
    x, xb = act(rng, M, k)
    y = run(F, fmt, bf16_dev(x), planes, 1)
    ref = og.matmul_f32(x, w_op) * np.float32(gs)
    print(f"{fmt} M={M}: max|d| {np.abs(to_f32(y) - ref).max():.3g}")
    assert_tol(to_f32(y), ref, what=f"{fmt} M={M}")
    # fp32 sums within the MFMA accumulation bound of the exact sum
    exact = ordered.exact_sum(x, w_op) * gs
    y32 = to_f32(run(F, fmt, bf16_dev(x), planes, 1, torch.float32))
    bound = ordered.mfma_bound(x, w_op) * abs(gs)
    assert np.all(np.abs(y32 - exact) <= bound), (np.abs(y32 - exact) / bound).max()
    print(f"{fmt} M={M}: max |y - exact| / bound = {(np.abs(y32 - exact) / bound).max():.3g}")


@pytest.mark.parametrize("fmt", ["mx8", "w8", "w8_f16", "w6", "nv4", "bf16"])
@pytest.mark.parametrize("N,M", [(512, 3), (512, 1), (512, 16), (96, 3), (1000, 4), (480, 8), (1024, 4), (200, 16),
                                 (1280, 3), (2048, 1), (1536, 4)])
def test_rows_gemv(gpu, F, fmt, N, M, monkeypatch):
    """Matrices whose 16-row tiles fill under half of the CUs (a router gate's
    512 x 2560) take the few-rows kernel (R rows per workgroup, one chunk per
    thread), and so do wider ones at M <= 4 whose one-row workgroups are all
    resident at once (1280, 2048 and 1536 rows): fp32 sums within the
    accumulation bound of the exact sums, equal to the other path's
    (FP4X_ROWS=0) within the two bounds, repeated calls bit for bit, bf16
    outputs the same sums rounded."""
    rng = np.random.default_rng(4000 + N + M)
    k = 2560
    base = "w8" if fmt == "w8_f16" else fmt
    planes, w_op, gs = prep(base, rng, N, k)
    if fmt == "w8_f16":
        q, s = planes
        s16 = s.half()
        planes = (q, s16)
        w_op = og.operand("w8", q.cpu().numpy(), s16.float().cpu().numpy())
    x, _ = act(rng, M, k)
    xd = bf16_dev(x)
    y = to_f32(run(F, base, xd, planes, 1, torch.float32))
    with path_switch(monkeypatch, "FP4X_ROWS"):
        y_core = to_f32(run(F, base, xd, planes, 1, torch.float32))
    if N * M >= 500:
        assert not np.array_equal(y.view(np.uint32), y_core.view(np.uint32)), "few-rows kernel not taken"
    exact = ordered.exact_sum(x, w_op) * gs
    bound = ordered.mfma_bound(x, w_op) * abs(gs)
    for got in (y, y_core):
        assert np.all(np.abs(got - exact) <= bound), (np.abs(got - exact) / bound).max()
    assert_tol(y, og.matmul_f32(x, w_op) * np.float32(gs), what=f"{fmt} rows N={N} M={M}")
    y2 = to_f32(run(F, base, xd, planes, 1, torch.float32))
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    yb = run(F, base, xd, planes, 1)
    assert np.array_equal(bf16_bits(yb), fm.bf16_bits(y))


@pytest.mark.parametrize("fmt", ["mx8", "w8", "w6", "nv4"])
@pytest.mark.parametrize("ks", [2, 4, 5])
def test_gemv_split_k(gpu, F, fmt, ks, monkeypatch):
    """K split over ks slices summed in slice order (the MFMA core and the
    split-K tile kernels; with FP4X_ROWS=0, since a 520-row matrix otherwise
    takes the few-rows kernels, which sum each row whole): within the bound,
    and repeated calls reuse the re-armed tickets bit for bit.  The default
    path is checked against the same bound."""
    rng = np.random.default_rng(7 + ks)
    n, k = 520, 2560
    planes, w_op, gs = prep(fmt, rng, n, k)
    x, xb = act(rng, 3, k)
    exact = ordered.exact_sum(x, w_op) * gs
    bound = ordered.mfma_bound(x, w_op, ks) * abs(gs)
    with path_switch(monkeypatch, "FP4X_ROWS"):
        y = run(F, fmt, bf16_dev(x), planes, ks, torch.float32)
        assert np.all(np.abs(to_f32(y) - exact) <= bound), (np.abs(to_f32(y) - exact) / bound).max()
        for _ in range(3):
            y2 = run(F, fmt, bf16_dev(x), planes, ks, torch.float32)
            assert torch.equal(y, y2)
    y3 = to_f32(run(F, fmt, bf16_dev(x), planes, ks, torch.float32))
    assert np.all(np.abs(y3 - exact) <= bound), (np.abs(y3 - exact) / bound).max()


@pytest.mark.parametrize("fmt", ["mx8", "w8", "w6", "nv4"])
@pytest.mark.parametrize("M", [16, 12])
def test_gemv_tile_groups(gpu, F, fmt, M):
    """Wide matrices at M = 16, where the activation stage leaves room for one
    workgroup per CU and each workgroup runs several tiles at once in wave
    groups (N = 8232: 515 tiles, so the last round of a workgroup has a
    padding group); M = 12 is the single-group control."""
    rng = np.random.default_rng(300 + M)
    n, k = 8232, 2560
    planes, w_op, gs = prep(fmt, rng, n, k)
    x, _ = act(rng, M, k)
    y = to_f32(run(F, fmt, bf16_dev(x), planes, 1, torch.float32))
    exact = ordered.exact_sum(x, w_op) * gs
    bound = ordered.mfma_bound(x, w_op) * abs(gs)
    assert np.all(np.abs(y - exact) <= bound), (np.abs(y - exact) / bound).max()
    assert_tol(y, og.matmul_f32(x, w_op) * np.float32(gs), what=f"{fmt} M={M}")
    y2 = to_f32(run(F, fmt, bf16_dev(x), planes, 1, torch.float32))
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("M", [1, 3, 16])
@pytest.mark.parametrize("tail", [0, 40])
@pytest.mark.parametrize("fmt,slots,parts,env", [("nv4", 4, 2, "FP4X_NV4_STREAM"), ("w6", 2, 2, "FP4X_W6_STREAM"),
                                                   ("mx8", 1, 10, "FP4X_MX8_STREAM")])
def test_dense_stream(gpu, F, fmt, slots, parts, env, M, tail, monkeypatch):
    """NVFP4 matrices of at least 4 tiles per CU (2 tile slots x 2 waves per
    workgroup at M <= 5, 4 x 2 above, a ring of 2 units of 256 K per wave), W6
    matrices of at least 2 (2 slots x 2 waves, 2 units of 256 K) and MXFP8
    matrices of at least 1 (1 slot x 10 waves, 2 units of 128 K) take the
    streaming kernel: fp32 sums within the MFMA
    bound of the exact sum, as the core's are; a 40-row tail leaves idle slots
    in the last workgroup (and, where two workgroups fit a CU, a second
    workgroup on some CUs).  K = 2560 runs the instantiation compiled for that
    row length."""
    _dense_stream_case(F, fmt, slots, parts, env, M, tail, 2560, monkeypatch)


@pytest.mark.parametrize("fmt,slots,parts,env", [("nv4", 8, 2, "FP4X_NV4_STREAM"), ("w6", 4, 2, "FP4X_W6_STREAM"),
                                                   ("mx8", 2, 10, "FP4X_MX8_STREAM")])
def test_dense_stream_rounds(gpu, F, fmt, slots, parts, env, monkeypatch):
    """Matrices past two workgroups per CU of one round each: workgroups of two
    rounds of T tiles, the last one's second round partly idle (a 40-row
    tail), against the same bound."""
    _dense_stream_case(F, fmt, slots, parts, env, 3, 40, 2560, monkeypatch)


@pytest.mark.parametrize("M", [1, 3])
@pytest.mark.parametrize("fmt,slots,parts,env", [("nv4", 4, 2, "FP4X_NV4_STREAM"), ("w6", 2, 2, "FP4X_W6_STREAM"),
                                                   ("mx8", 1, 10, "FP4X_MX8_STREAM")])
def test_dense_stream_other_k(gpu, F, fmt, slots, parts, env, M, monkeypatch):
    """K = 5120: the streaming kernels' instantiation that reads the row
    length at run time (twice the units per wave), against the same bound."""
    _dense_stream_case(F, fmt, slots, parts, env, M, 40, 5120, monkeypatch)


@pytest.mark.parametrize("fmt,slots,M,env", [
    ("nv4", 2, 3, "FP4X_NV4_STREAM"),    # 2 to 4 tiles per CU: 2 slots x 2 waves
    ("nv4", 2, 8, "FP4X_NV4_STREAM"),
    ("nv4", 1, 8, "FP4X_NV4_STREAM"),    # 1 to 2 tiles per CU: one slot, two workgroups per CU
    ("w6", 1, 8, "FP4X_W6_STREAM"),
    ("w6", 1.5, 3, "FP4X_W6_STREAM"),
])
def test_dense_stream_mid(gpu, F, fmt, slots, M, env, monkeypatch):
    """NVFP4 matrices of 2 to 4 tiles per CU, and W6 / NVFP4 matrices of 1 to 2
    tiles per CU that the few-rows kernel leaves (M >= 5, or past its limits)
    stream with fewer tile slots per workgroup, against the same bound."""
    _dense_stream_case(F, fmt, slots, 2, env, M, 40, 2560, monkeypatch)


@pytest.mark.parametrize("fmt,slots,k,M,parts,env", [
    ("w6", 0.625, 6144, 5, 8, "FP4X_W6_STREAM"),      # [2600 x 6144]: 8 waves of 3 units per tile
    ("nv4", 0.625, 6144, 8, 8, "FP4X_NV4_STREAM"),
    ("mx8", 0.625, 6144, 5, 8, "FP4X_MX8_STREAM"),    # 8 waves of 6 128-K units
    ("w6", 0.5, 2560, 16, 5, "FP4X_W6_STREAM"),       # [2088 x 2560]: 5 waves of 2 units
    ("nv4", 0.5, 2560, 5, 5, "FP4X_NV4_STREAM"),
    ("mx8", 0.5, 2560, 8, 5, "FP4X_MX8_STREAM"),
])
def test_dense_stream_tile_per_workgroup(gpu, F, fmt, slots, k, M, parts, env, monkeypatch):
    """Matrices of half a tile to one tile per CU at M >= 5 (the few-rows kernel
    takes M <= 4): one tile per workgroup, its K over `parts` waves, against
    the same bound."""
    _dense_stream_case(F, fmt, slots, parts, env, M, 40, k, monkeypatch)


def _dense_stream_case(F, fmt, slots, parts, env, M, tail, k, monkeypatch):
    rng = np.random.default_rng(500 + M + tail + int(2 * slots) + k)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    n = int(16 * slots * cus) + tail
    planes, w_op, gs = prep(fmt, rng, n, k)
    x, _ = act(rng, M, k)
    with path_switch(monkeypatch, "FP4X_ROWS"):        # MXFP8 at M <= 2 takes the few-rows kernel first
        y = to_f32(run(F, fmt, bf16_dev(x), planes, 1, torch.float32))
        with path_switch(monkeypatch, env):
            y_core = to_f32(run(F, fmt, bf16_dev(x), planes, 1, torch.float32))
        yb = run(F, fmt, bf16_dev(x), planes, 1)                    # bf16 output: the same sums rounded
    assert not np.array_equal(y.view(np.uint32), y_core.view(np.uint32)), "streaming kernel not taken"
    exact = ordered.exact_sum(x, w_op) * gs
    bound = ordered.mfma_bound(x, w_op, parts) * abs(gs)              # parts: K slices of a tile
    for got in (y, y_core):
        assert np.all(np.abs(got - exact) <= bound), (np.abs(got - exact) / bound).max()
    assert_tol(y, og.matmul_f32(x, w_op) * np.float32(gs), what=f"{fmt} stream M={M}")
    assert np.array_equal(bf16_bits(yb), fm.bf16_bits(y))


@pytest.mark.parametrize("case", [
    # tiles as a multiple of the CUs (or N), K, M, scale dtype, waves per tile
    ((4, 40), 2560, 3, np.float32, 2),    # 4 tile slots x 2 waves, a 40-row tail
    ((4, 0), 2560, 16, np.float16, 2),
    (13312, 2560, 3, np.float32, 2),       # the MTP attention qkv: 2 slots x 2 waves
    (13312, 2560, 1, np.float16, 2),
    ((1, 40), 2560, 3, np.float32, 5),    # one tile per workgroup, 5 waves of 2 units
    ((1, 0), 2560, 16, np.float16, 5),
    (2560, 6144, 3, np.float32, 12),       # the MTP attention output: 12 waves of 2 units
    (2560, 6144, 5, np.float32, 8),        # its activations leave room for 8 waves of 3 units
    (2560, 6144, 8, np.float16, 4),        # ... and for 4 waves of 6 units
    (2048, 4096, 5, np.float16, 4),        # K = 4096 (run-time K): 4 waves of 4 units
])
def test_w8_single_stream(gpu, F, case, monkeypatch):
    """Single W8 matrices without split-K of at least half a tile per CU stream
    through LDS (fp32 or fp16 scales), with the few-rows kernels off
    (FP4X_ROWS=0; at M <= 4 they take some of these shapes first): fp32 sums
    within the MFMA bound of the exact sum (the tile's K over `parts` waves),
    a different K decomposition than the MFMA core's (FP4X_W8_STREAM=0),
    repeated calls bit for bit, bf16 outputs the same sums rounded."""
    size, k, M, s_dtype, parts = case
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    n = 16 * size[0] * cus + size[1] if isinstance(size, tuple) else size
    rng = np.random.default_rng(5000 + n + k + M)
    q, s = oq.quantize_w8(weights(rng, n, k))
    s = s.astype(s_dtype)
    x, _ = act(rng, M, k)
    qd, sd, xd = dev(q), dev(s), bf16_dev(x)
    w_op = og.operand("w8", q, s.astype(np.float32))
    with path_switch(monkeypatch, "FP4X_ROWS"):
        y = to_f32(F.w8_linear(xd, qd, sd, (32, 256, 1, 4), torch.float32))
        with path_switch(monkeypatch, "FP4X_W8_STREAM"):
            y_core = to_f32(F.w8_linear(xd, qd, sd, (32, 256, 1, 4), torch.float32))
        y2 = to_f32(F.w8_linear(xd, qd, sd, (32, 256, 1, 4), torch.float32))
        yb = F.w8_linear(xd, qd, sd, (32, 256, 1, 4))
    assert not np.array_equal(y.view(np.uint32), y_core.view(np.uint32)), "streaming kernel not taken"
    exact = ordered.exact_sum(x, w_op)
    bound = ordered.mfma_bound(x, w_op, parts)
    for got in (y, y_core):
        assert np.all(np.abs(got - exact) <= bound), (np.abs(got - exact) / bound).max()
    assert_tol(y, og.matmul_f32(x, w_op), what=f"w8 single stream N={n} K={k} M={M}")
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    assert np.array_equal(bf16_bits(yb), fm.bf16_bits(y))
    print(f"N={n} K={k} M={M} {np.dtype(s_dtype).name}: max |y - exact| / bound = "
          f"{(np.abs(y - exact) / bound).max():.3g}")


@pytest.mark.parametrize("case", [
    # N, K, M, ksplit, scale dtype, split over workgroups
    (640, 10240, 3, 4, np.float16, True),    # the mixer's down projection: 5 workgroups per tile
    (640, 10240, 1, 4, np.float32, True),
    (1000, 4096, 5, 2, np.float32, True),    # N tail (rows past N), M > 4, 2 workgroups per tile
    (520, 8192, 16, 8, np.float16, True),    # M = 16 (the last workgroup sums 256 outputs)
    (520, 8192, 16, 4, np.float16, False),   # the slots exceed ksplit = 4's scratch: the MFMA core
])
def test_w8_splitk_workgroups(gpu, F, case, monkeypatch):
    """W8 split-K of few tiles with K a multiple of 2048: each tile's K spread over
    several workgroups, partials summed in slot order by the last one to arrive
    (FP4X_ROWS=0: these shapes otherwise take the few-rows kernels)."""
    n, k, M, ks, s_dtype, split = case
    rng = np.random.default_rng(2000 + n + k + M + ks)
    q, s = oq.quantize_w8(weights(rng, n, k))
    s = s.astype(s_dtype)
    x, _ = act(rng, M, k)
    qd, sd, xd = dev(q), dev(s), bf16_dev(x)
    w_op = og.operand("w8", q, s.astype(np.float32))
    exact = ordered.exact_sum(x, w_op)
    bound = ordered.mfma_bound(x, w_op, max(ks, k // 2048))
    with path_switch(monkeypatch, "FP4X_ROWS"):
        y = F.w8_linear(xd, qd, sd, (32, 64, ks, 4), torch.float32)
        assert np.all(np.abs(to_f32(y) - exact) <= bound), (np.abs(to_f32(y) - exact) / bound).max()
        assert_tol(to_f32(y), og.matmul_f32(x, w_op), what=str(case))
        for _ in range(3):                        # re-armed tickets, arrival order does not matter
            assert torch.equal(y, F.w8_linear(xd, qd, sd, (32, 64, ks, 4), torch.float32))
        with path_switch(monkeypatch, "FP4X_W8_STREAM"):
            y_core = F.w8_linear(xd, qd, sd, (32, 64, ks, 4), torch.float32)
    assert np.all(np.abs(to_f32(y_core) - exact) <= bound)
    # another K decomposition than the core's: its fp32 sums differ in the last bits
    assert (not torch.equal(y, y_core)) == split
    print(f"N={n} K={k} M={M} ksplit={ks}: split={split}, max |y - exact| / bound = "
          f"{(np.abs(to_f32(y) - exact) / bound).max():.3g}")
    # the default path (few-rows kernels where they apply) within the same bound
    y_def = to_f32(F.w8_linear(xd, qd, sd, (32, 64, ks, 4), torch.float32))
    assert np.all(np.abs(y_def - exact) <= bound), (np.abs(y_def - exact) / bound).max()


def test_gemv_out_dtypes_and_strided_x(gpu, F):
    rng = np.random.default_rng(5)
    planes, w_op, _ = prep("mx8", rng, 256, 512)
    x, _ = act(rng, 4, 1024)
    xt = bf16_dev(x)[:, 256:768]                     # row stride 1024, offset view
    ref = og.matmul_f32(x[:, 256:768], w_op)
    for dt in (torch.bfloat16, torch.float32, torch.float16):
        y = F.mx8_linear(xt, *planes, (32, 64, 1, 4), dt)
        assert y.dtype == dt
        assert_tol(to_f32(y), ref, what=str(dt))


@pytest.mark.parametrize("fmt,rows,k,M", [
    ("w6", (10, 0), 6144, 3),      # few-rows kernel, 2 rows per workgroup, two lanes per chunk
    ("mx8", (10, 0), 6144, 1),     # few-rows kernel, 2 rows per workgroup, rows of 384 chunks
    ("w6", (32, 8), 2560, 1),      # W6 ahead of its streaming kernel
    ("mx8", (16, 0), 2560, 3),     # streaming, 5 waves per tile
    ("nv4", (32, 40), 2560, 3),    # streaming, 2 slots, two workgroups per CU
    ("w6", (10, 0), 6144, 5),      # one tile per workgroup, 8 waves
    ("w8", (52, 0), 2560, 3),      # W8 single-matrix streaming, 2 slots
])
def test_gemv_strided_x_paths(gpu, F, fmt, rows, k, M):
    """Activations as an offset column slice of a wider tensor (row stride K +
    512, 16-byte aligned) on each dispatch path: the same results as from a
    contiguous copy, bit for bit, and within the tolerance of the oracle."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    n = rows[0] * cus + rows[1]
    rng = np.random.default_rng(6100 + n + k + M)
    planes, w_op, gs = prep(fmt, rng, n, k)
    x, _ = act(rng, M, k + 512)
    wide = bf16_dev(x)
    xt = wide[:, 256:256 + k]                        # row stride k + 512, offset 512 bytes
    y = to_f32(run(F, fmt, xt, planes, 1, torch.float32))
    y_c = to_f32(run(F, fmt, xt.contiguous(), planes, 1, torch.float32))
    assert np.array_equal(y.view(np.uint32), y_c.view(np.uint32))
    assert_tol(y, og.matmul_f32(x[:, 256:256 + k], w_op) * np.float32(gs), what=f"{fmt} strided N={n} M={M}")


def test_gemv_shape_errors(gpu, F):
    rng = np.random.default_rng(6)
    planes, _, _ = prep("mx8", rng, 64, 512)
    x = bf16_dev(act(rng, 2, 512)[0])
    with pytest.raises(AssertionError):
        F.mx8_linear(x, *planes, (32, 512, 3, 4))     # K not divisible by KSPLIT*BK (reference precondition)
    with pytest.raises(TypeError):
        F.mx8_linear(x.float(), *planes, (32, 64, 1, 4))
    y = F.mx8_linear(x[:0], *planes, (32, 64, 1, 4))
    assert y.shape == (0, 64)


@pytest.mark.parametrize("N,K,M", [(10240, 320, 3), (10240, 640, 3), (10240, 320, 1)])
def test_mixer_up_shape_takes_the_core(gpu, F, N, K, M, monkeypatch):
    """The mixer's up projection [10240 x 320 or 640] through w8_linear (the
    unfused mixer's gate logits) stays on the MFMA core, bit for bit with
    FP4X_ROWS=0, so that the unfused mixer equals the single-launch one."""
    rng = np.random.default_rng(4300 + N + K + M)
    q, s = oq.quantize_w8(weights(rng, N, K))
    x, _ = act(rng, M, K)
    xd, qd, sd = bf16_dev(x), dev(q), dev(s)
    y = F.w8_linear(xd, qd, sd, (32, 64, 1, 4), torch.float32)
    with path_switch(monkeypatch, "FP4X_ROWS"):
        y_core = F.w8_linear(xd, qd, sd, (32, 64, 1, 4), torch.float32)
    assert torch.equal(y, y_core)


@pytest.mark.parametrize("N,K,M", [(2560, 640, 3), (2560, 640, 1), (4096, 640, 4), (2560, 1280, 2)])
def test_rows_gemv_short_rows(gpu, F, N, K, M, monkeypatch):
    """W8 matrices of short rows (the MTP shared expert's down projection,
    [2560 x 640]) take the fma few-rows kernel, one row per workgroup: the same
    checks as above against the MFMA core (FP4X_ROWS=0)."""
    rng = np.random.default_rng(4100 + N + K + M)
    q, s = oq.quantize_w8(weights(rng, N, K))
    x, _ = act(rng, M, K)
    xd, qd, sd = bf16_dev(x), dev(q), dev(s)
    w_op = og.operand("w8", q, s)
    cfg = (32, 64, 1, 4)
    y = to_f32(F.w8_linear(xd, qd, sd, cfg, torch.float32))
    with path_switch(monkeypatch, "FP4X_ROWS"):
        y_core = to_f32(F.w8_linear(xd, qd, sd, cfg, torch.float32))
    assert not np.array_equal(y.view(np.uint32), y_core.view(np.uint32)), "few-rows kernel not taken"
    exact = ordered.exact_sum(x, w_op)
    bound = ordered.mfma_bound(x, w_op)
    for got in (y, y_core):
        assert np.all(np.abs(got - exact) <= bound), (np.abs(got - exact) / bound).max()
    assert_tol(y, og.matmul_f32(x, w_op), what=f"w8 rows N={N} K={K} M={M}")
    assert np.array_equal(y.view(np.uint32), to_f32(F.w8_linear(xd, qd, sd, cfg, torch.float32)).view(np.uint32))
    assert np.array_equal(bf16_bits(F.w8_linear(xd, qd, sd, cfg)), fm.bf16_bits(y))


@pytest.mark.parametrize("fmt", ["mx8", "w8", "w8_f16", "w6", "nv4", "bf16"])
@pytest.mark.parametrize("rows,K,M", [
    # rows as (multiple of the CUs, extra rows)
    ((10, 0), 6144, 3),      # the attention output projection [2560 x 6144]: 2 rows per workgroup (MXFP8 and NVFP4 stream)
    ((10, 0), 6144, 1),      # M = 1: W6 / NVFP4 one row per workgroup, the 384-chunk formats 2
    ((8, 1), 2560, 4),       # an odd N: the last workgroup's second row lies past N
    ((16, 1), 2560, 2),      # 2 rows per workgroup (MXFP8 streams at M = 2), N odd
    ((16, 0), 2560, 1),      # MXFP8 [4096 x 2560] at M = 1: 2 rows per workgroup
    ((10, 0), 2560, 4),      # MXFP8 and NVFP4 stream at M = 4 from 10 rows per CU
])
def test_rows_gemv_multi(gpu, F, fmt, rows, K, M, monkeypatch):
    """Matrices of at least 8 rows per CU at M = 2..4, and of rows past the
    one-row kernel's limits, take the fma few-rows kernel with R = 2 rows per
    workgroup (MXFP8 [4096 x 2560] at M = 1 too), except where MXFP8 and
    NVFP4 stream (10 rows per CU or more at M >= 3 with K >= 4096 and at
    M = 4; MXFP8 from 16 rows per CU at M >= 2), which must then equal the
    FP4X_ROWS=0 path: fp32 sums
    within the accumulation bound of the exact sums and different from the
    other path's (FP4X_ROWS=0; both within the bound), repeated calls bit for
    bit, bf16 outputs the same sums rounded."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    N = rows[0] * cus + rows[1]
    rng = np.random.default_rng(4500 + N + K + M)
    base = "w8" if fmt == "w8_f16" else fmt
    planes, w_op, gs = prep(base, rng, N, K)
    if fmt == "w8_f16":
        q, s = planes
        s16 = s.half()
        planes = (q, s16)
        w_op = og.operand("w8", q.cpu().numpy(), s16.float().cpu().numpy())
    x, _ = act(rng, M, K)
    xd = bf16_dev(x)
    print(f"{fmt} N={N} K={K} M={M}", flush=True)
    y = to_f32(run(F, base, xd, planes, 1, torch.float32))
    with path_switch(monkeypatch, "FP4X_ROWS"):
        y_other = to_f32(run(F, base, xd, planes, 1, torch.float32))
    # MXFP8 and NVFP4 stream from 10 rows per CU at M >= 3 with K >= 4096 and
    # at M = 4, MXFP8 from 16 rows per CU at M >= 2: the same sums as with the
    # few-rows kernels off
    streams = (base in ("mx8", "nv4") and M >= 3 and N >= 10 * cus and (K >= 4096 or M >= 4)) or \
        (base == "mx8" and M >= 2 and N >= 16 * cus)
    if streams:
        assert np.array_equal(y.view(np.uint32), y_other.view(np.uint32)), "streaming path not taken"
    else:
        assert not np.array_equal(y.view(np.uint32), y_other.view(np.uint32)), "few-rows kernel not taken"
    exact = ordered.exact_sum(x, w_op) * gs
    for got, parts in ((y, 12 if streams else 1), (y_other, 12)):
        bound = ordered.mfma_bound(x, w_op, parts) * abs(gs)
        assert np.all(np.abs(got - exact) <= bound), (np.abs(got - exact) / bound).max()
    assert_tol(y, og.matmul_f32(x, w_op) * np.float32(gs), what=f"{fmt} rows N={N} K={K} M={M}")
    y2 = to_f32(run(F, base, xd, planes, 1, torch.float32))
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    yb = run(F, base, xd, planes, 1)
    assert np.array_equal(bf16_bits(yb), fm.bf16_bits(y))


@pytest.mark.parametrize("rows", [(32, 8), (52, 0)])
def test_rows_w6_wide(gpu, F, rows, monkeypatch):
    """W6 at M = 1 with 32 to 52 rows per CU takes the few-rows kernel (2 rows
    per workgroup, two lanes per chunk, several rounds) ahead of the streaming
    kernel: the same checks as test_rows_gemv_multi."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    N, K, M = rows[0] * cus + rows[1], 2560, 1
    rng = np.random.default_rng(4700 + N)
    planes, w_op, gs = prep("w6", rng, N, K)
    x, _ = act(rng, M, K)
    xd = bf16_dev(x)
    print(f"w6 N={N} K={K} M={M}", flush=True)
    y = to_f32(run(F, "w6", xd, planes, 1, torch.float32))
    with path_switch(monkeypatch, "FP4X_ROWS"):
        y_other = to_f32(run(F, "w6", xd, planes, 1, torch.float32))
    assert not np.array_equal(y.view(np.uint32), y_other.view(np.uint32)), "few-rows kernel not taken"
    exact = ordered.exact_sum(x, w_op)
    for got, parts in ((y, 1), (y_other, 2)):
        bound = ordered.mfma_bound(x, w_op, parts)
        assert np.all(np.abs(got - exact) <= bound), (np.abs(got - exact) / bound).max()
    assert_tol(y, og.matmul_f32(x, w_op), what=f"w6 wide rows N={N}")
    assert np.array_equal(y.view(np.uint32), to_f32(run(F, "w6", xd, planes, 1, torch.float32)).view(np.uint32))


def test_w8_fp16_scales_and_layers(gpu, F):
    rng = np.random.default_rng(9)
    Ly, n, k, M = 6, 512, 2560, 3
    ws = [weights(rng, n, k) for _ in range(Ly)]
    qs = [oq.quantize_w8(w) for w in ws]
    xs = [act(rng, M, k)[0] for _ in range(Ly)]
    for s_dtype in (np.float32, np.float16):
        q3 = dev(np.stack([q for q, _ in qs]))
        s3 = dev(np.stack([s.astype(s_dtype) for _, s in qs]))
        x3 = bf16_dev(np.stack(xs))
        y = F.w8_linear_layers(x3, q3, s3, torch.float32)
        for i in range(Ly):
            w_op = og.operand("w8", qs[i][0], qs[i][1].astype(s_dtype).astype(np.float32))
            ref = og.matmul_f32(xs[i], w_op)
            assert_tol(to_f32(y[i]), ref, what=f"layer {i}")
            # the single-layer call (the few-rows kernel) sums in another fixed
            # order: both within the accumulation bound of the exact sums, and
            # the single call repeats bit for bit
            single = F.w8_linear(x3[i], q3[i], s3[i], (16, 512, 1, 4), torch.float32)
            exact, bound = ordered.exact_sum(xs[i], w_op), ordered.mfma_bound(xs[i], w_op)
            for got in (to_f32(single), to_f32(y[i])):
                assert np.all(np.abs(got - exact) <= bound), (np.abs(got - exact) / bound).max()
            assert torch.equal(single, F.w8_linear(x3[i], q3[i], s3[i], (16, 512, 1, 4), torch.float32))


# ------------------------------------------------------------------ streaming W8 (layer-batched gates)
@pytest.mark.parametrize("case", [
    # layers, N, K, M, scale dtype
    (48, 512, 2560, 3, np.float16),    # the router-gate workload: one round of 6 tiles per CU
    (48, 512, 2560, 3, np.float32),
    (48, 512, 2560, 1, np.float32),
    (40, 512, 2560, 5, np.float16),    # fewer tiles than CUs x 6: falls back to the MFMA core
    (96, 512, 2560, 3, np.float16),    # two rounds per workgroup: the ring crosses tiles
    (25, 1000, 2560, 3, np.float32),   # N tail (rows past N) and idle slots in the last round
    (48, 512, 1024, 2, np.float16),    # K = 1024: 4 units per wave
])
def test_w8_stream_layers(gpu, F, case, monkeypatch):
    Ly, n, k, M, s_dtype = case
    rng = np.random.default_rng(1000 + Ly + n + k + M)
    q3n = np.empty((Ly, n, k), np.int8)
    s3n = np.empty((Ly, n, k // 64), np.float32)
    for i in range(Ly):
        q3n[i], s3n[i] = oq.quantize_w8(weights(rng, n, k))
    s3n = s3n.astype(s_dtype)
    x3n = np.stack([act(rng, M, k)[0] for _ in range(Ly)])
    q3, s3, x3 = dev(q3n), dev(s3n), bf16_dev(x3n)
    y = to_f32(F.w8_linear_layers(x3, q3, s3, torch.float32))
    with path_switch(monkeypatch, "FP4X_W8_STREAM"):
        y_core = to_f32(F.w8_linear_layers(x3, q3, s3, torch.float32))
    worst = 0.0
    for i in range(Ly):
        w_op = og.operand("w8", q3n[i], s3n[i].astype(np.float32))
        ref = og.matmul_f32(x3n[i], w_op)
        assert_tol(y[i], ref, what=f"layer {i}")
        exact = ordered.exact_sum(x3n[i], w_op)
        bound = ordered.mfma_bound(x3n[i], w_op)
        assert np.all(np.abs(y[i] - exact) <= bound), (i, (np.abs(y[i] - exact) / bound).max())
        assert np.all(np.abs(y_core[i] - exact) <= bound)
        worst = max(worst, float((np.abs(y[i] - exact) / bound).max()))
    streamed = not np.array_equal(y.view(np.uint32), y_core.view(np.uint32))
    print(f"layers={Ly} N={n} K={k} M={M} {np.dtype(s_dtype).name}: streamed={streamed}, "
          f"max |y - exact| / bound = {worst:.3g}")
    # the workload shapes above the CUs x 6 tile threshold take the streaming kernel (a different
    # K decomposition, so its fp32 sums differ from the core's in the last bits)
    assert streamed == (Ly * ((n + 15) // 16) >= 6 * torch.cuda.get_device_properties(0).multi_processor_count)
