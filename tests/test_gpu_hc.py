"""GPU parity of the hyper-connection mixer kernels.

* fused (hc_down + hc_up), single-launch (HCFused.mix) and unfused (W8 GEMV,
  scaled SiLU, W8 GEMV, gate mean) agree bit for bit, over all 97 seeded
  layers at the synthetic shape (x [3, 4 x 2560], W_down [640, 10240], W_up
  [10240, 640], 16 K-splits), and the scratch is re-armed after every call;
* against the oracle, split at its two sources of difference:
  - the GEMV sums (di, and the gate logits g of the unfused path) lie within
    the MFMA accumulation bound of the exact sums, plus half a bf16 ulp;
  - the epilogues are bit-exact on the kernel's own GEMV outputs:
    bot = oracle.scaled_silu(di), block_input = oracle.gate_mean(x, g)
    (the device sigmoid is the correctly rounded fp32 one, as the oracle's);
  - end to end, block_input against the oracle's mixer (numpy fp32 GEMVs)
    stays within the GEMV bar plus one bf16 ulp of the output; the
    bit-agreement rate is printed;
* the epilogue kernels equal the oracle bit for bit on every finite bf16
  input;
* a single-launch call whose flag wait gives up (forced from the host with
  FP4X_HC_SPIN_LIMIT=0) writes NaN and sets the status word, and the next
  call is bit-identical to the two-launch path;
* single-launch calls whose up workgroups get a CU only after the bottleneck
  is ready (a kernel on another stream holds most CUs) are bit-identical to
  the two-launch path, with no NaN and no status bit;
* single launches whose down tiles split into 2 and 8 K parts (hidden sizes
  1024 and 4096), whose closers add 1 and 7 other parts' tagged partials,
  are bit-identical to the two-launch path;
* single launches of different row counts and batch sizes that share one
  scratch are bit-identical to the two-launch path.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import formats as fm
from oracle import hc as ohc
from oracle import ordered
from oracle import quant as oq

from gpu_helpers import act, bf16_bits, bf16_dev, dev, to_f32, path_switch

pytestmark = pytest.mark.gpu

HC, H, LR, ND, KS = 4, 2560, 640, 640, 16


@pytest.fixture(scope="module")
def F():
    import fp4x_kernels
    return fp4x_kernels


def layer(rng, nd=ND, lr=LR, h=H):
    wd = (rng.standard_normal((nd, HC * h)) * 0.02).astype(np.float32)
    wu = (rng.standard_normal((HC * h, lr)) * 0.02).astype(np.float32)
    return oq.quantize_w8(wd), oq.quantize_w8(wu)


def unfused(F, x_t, qd, sd, qu, su, lr, ks):
    di = F.w8_linear(x_t, qd, sd, (32, 64, ks, 4))
    bot = F.hc_scaled_silu(di, lr, HC)
    g = F.w8_linear(bot, qu, su, (32, 64, 1, 4))
    return di, bot, F.hc_gate_mean(x_t, g, HC), g


def ulp_bf16(v):
    """One bf16 ulp at |v| (the spacing above |v|'s binade start)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 2.0 ** -126)))
    return 2.0 ** (np.maximum(e, -126) - 7)


def check_against_oracle(x, qd, sd, qu, su, lr, di, bot, g, bi, ks, what):
    """The four oracle checks of one mixer call; returns the bit agreement of
    block_input with the oracle's mixer."""
    wd = fm.round_bf16(oq.dequant_w8(qd, sd))
    exact = ordered.exact_sum(x, wd)
    bound = ordered.mfma_bound(x, wd, ks) + np.abs(exact) * 2.0 ** -8
    assert np.all(np.abs(to_f32(di) - exact) <= bound), f"{what}: di"
    assert np.array_equal(bf16_bits(bot), fm.bf16_bits(ohc.scaled_silu(to_f32(di)[:, :lr], HC))), f"{what}: bot"
    wu = fm.round_bf16(oq.dequant_w8(qu, su))
    b32 = to_f32(bot)
    exact_g = ordered.exact_sum(b32, wu)
    bound_g = ordered.mfma_bound(b32, wu) + np.abs(exact_g) * 2.0 ** -8
    assert np.all(np.abs(to_f32(g) - exact_g) <= bound_g), f"{what}: gate logits"
    assert np.array_equal(bf16_bits(bi), fm.bf16_bits(ohc.gate_mean(x, to_f32(g), HC))), f"{what}: block_input"
    _, _, bi_ref = ohc.mixer(x, qd, sd, qu, su, lr, HC)
    got = to_f32(bi).astype(np.float64)
    tol = 1e-2 + 2e-3 * np.abs(bi_ref) + ulp_bf16(bi_ref)
    assert np.all(np.abs(got - bi_ref) <= tol), (f"{what}: block_input vs the oracle mixer, max |d| "
                                                f"{np.abs(got - bi_ref).max():.3g}")
    return float((bf16_bits(bi) == fm.bf16_bits(bi_ref)).mean())


def test_fused_equals_unfused_97_layers(gpu, F):
    rng = np.random.default_rng(2024)
    gen = torch.Generator(device=gpu).manual_seed(2024)
    fx = F.HCFused(gpu, n_down=ND, max_ksplit=KS)
    x, xb = act(rng, 3, HC * H)
    x_t = bf16_dev(x)
    agree = []
    for i in range(97):
        wd = torch.randn((ND, HC * H), generator=gen, device=gpu) * 0.02
        wu = torch.randn((HC * H, LR), generator=gen, device=gpu) * 0.02
        qd_t, sd_t = F.quantize_w8(wd)
        qu_t, su_t = F.quantize_w8(wu)
        qi, si = F.HCFused.interleave_up(qu_t, su_t, HC, 8)
        di, bot = fx.down(x_t, qd_t, sd_t, LR, HC, (32, 256, KS, 4))
        bi = F.HCFused.up(bot, qi, si, x_t, HC, (8, 64, 4))
        di2, bot2, bi2, g = unfused(F, x_t, qd_t, sd_t, qu_t, su_t, LR, KS)
        assert torch.equal(di, di2) and torch.equal(bot, bot2) and torch.equal(bi, bi2), f"layer {i}"
        assert int(fx.tickets[:fx._status_at].abs().sum()) == 0
        di3, bot3, bi3 = fx.mix(x_t, qd_t, sd_t, LR, HC, qi, si, x_t, (32, 256, KS, 4))
        assert torch.equal(di, di3) and torch.equal(bot, bot3) and torch.equal(bi, bi3), f"layer {i} mix"
        qd, sd, qu, su = (t.cpu().numpy() for t in (qd_t, sd_t, qu_t, su_t))
        agree.append(check_against_oracle(x, qd, sd, qu, su, LR, di, bot, g, bi, KS, f"layer {i}"))
    assert not fx.wait_timeouts()
    print(f"block_input bit agreement with the oracle mixer over 97 layers: mean {np.mean(agree):.5f}, "
          f"min {np.min(agree):.5f}")


@pytest.mark.parametrize("M", [1, 3, 8, 16])
def test_mixer_served_shape(gpu, F, M):
    """Served shape: down [336, 10240] (320 bottleneck + 4 injection rows + pad), up [10240, 320]."""
    rng = np.random.default_rng(M)
    (qd, sd), (qu, su) = layer(rng, nd=336, lr=320)
    x, _ = act(rng, M, HC * H)
    x_t = bf16_dev(x)
    fx = F.HCFused(gpu)
    qi, si = F.HCFused.interleave_up(dev(qu), dev(su), HC, 8)
    di, bot = fx.down(x_t, dev(qd), dev(sd), 320, HC, (32, 256, 8, 4))
    bi = F.HCFused.up(bot, qi, si, x_t, HC, (8, 64, 4))
    di2, bot2, bi2, g = unfused(F, x_t, dev(qd), dev(sd), dev(qu), dev(su), 320, 8)
    assert torch.equal(di, di2) and torch.equal(bot, bot2) and torch.equal(bi, bi2)
    for _ in range(3):                                # one launch, counters re-armed every call
        di3, bot3, bi3 = fx.mix(x_t, dev(qd), dev(sd), 320, HC, qi, si, x_t, (32, 256, 8, 4))
        assert torch.equal(di, di3) and torch.equal(bot, bot3) and torch.equal(bi, bi3)
        assert int(fx.tickets[:fx._status_at].abs().sum()) == 0
    agree = check_against_oracle(x, qd, sd, qu, su, 320, di, bot, g, bi, 8, f"M={M}")
    print(f"served shape M={M}: block_input bit agreement with the oracle mixer {agree:.5f}")


def all_finite_bf16():
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    return b[(b & 0x7F80) != 0x7F80]


@pytest.mark.parametrize("hc", [4, 3, 1])
def test_scaled_silu_kernel_every_bf16(gpu, F, hc):
    """fp4x_hc_scaled_silu on every finite bf16 input equals the oracle bit for
    bit (hc = 1: the output is bf16(sc * sigmoid(sc)) itself, for every bf16
    sc)."""
    bits = all_finite_bf16()
    n = bits.size // 64 * 64
    d = fm.bf16_to_f32(bits[:n]).reshape(64, -1)
    got = F.hc_scaled_silu(bf16_dev(d), d.shape[1], hc)
    want = ohc.scaled_silu(d, hc)
    assert np.array_equal(bf16_bits(got), fm.bf16_bits(want))


def test_gate_mean_kernel_every_bf16(gpu, F):
    """fp4x_hc_gate_mean with every finite bf16 gate logit (four streams per
    output, random bf16 normalized inputs) equals the oracle bit for bit."""
    rng = np.random.default_rng(11)
    bits = all_finite_bf16()
    Hh = bits.size // HC
    g = fm.bf16_to_f32(rng.permutation(bits)[:HC * Hh]).reshape(1, HC * Hh)
    g = np.repeat(g, 2, 0)
    nrm = fm.round_bf16((rng.standard_normal((2, HC * Hh)) * 2).astype(np.float32))
    got = F.hc_gate_mean(bf16_dev(nrm), bf16_dev(g), HC)
    want = ohc.gate_mean(nrm, g, HC)
    assert np.array_equal(bf16_bits(got), fm.bf16_bits(want))


def test_gate_every_bf16_logit(gpu, F):
    """One stream (hc = 1) and normalized inputs of 1: the gate-mean output is
    bf16(sigmoid(g)) itself, for every finite bf16 gate logit, bit for bit with
    the oracle."""
    bits = all_finite_bf16()
    g = fm.bf16_to_f32(bits).reshape(2, -1)
    nrm = np.ones_like(g)
    got = F.hc_gate_mean(bf16_dev(nrm), bf16_dev(g), 1)
    want = ohc.gate_mean(nrm, g, 1)
    assert np.array_equal(bf16_bits(got), fm.bf16_bits(want))
    assert np.array_equal(fm.bf16_bits(want), fm.bf16_bits(ohc.round_bf16(ohc.sigmoid32(g))))


def f16_w8(w):
    g = w.reshape(w.shape[0], -1, 64)
    s16 = (g.abs().amax(-1).clamp_min(1e-12) / 127.0).half()
    q = torch.round(g / s16.float().unsqueeze(-1)).clamp(-127, 127).to(torch.int8).reshape(w.shape)
    return q.contiguous(), s16.contiguous()


def test_mix_fallback_and_fp16_scales(gpu, F, monkeypatch):
    """The two-call fallback (FP4X_HC_MIX=0) and the single launch agree, with
    fp16 scales, across repeated calls sharing one scratch."""
    rng = np.random.default_rng(77)
    gen = torch.Generator(device=gpu).manual_seed(77)
    wd = torch.randn((336, HC * H), generator=gen, device=gpu) * 0.02
    wu = torch.randn((HC * H, 320), generator=gen, device=gpu) * 0.02
    qd, sd = f16_w8(wd)
    qu, su = f16_w8(wu)
    qi, si = F.HCFused.interleave_up(qu, su, HC, 8)
    fx = F.HCFused(gpu)
    for M in (3, 16, 1):
        x_t = bf16_dev(act(rng, M, HC * H)[0])
        one = fx.mix(x_t, qd, sd, 320, HC, qi, si, x_t, (32, 256, 8, 4))
        with path_switch(monkeypatch, "FP4X_HC_MIX"):
            two = fx.mix(x_t, qd, sd, 320, HC, qi, si, x_t, (32, 256, 8, 4))
        di, bot = fx.down(x_t, qd, sd, 320, HC, (32, 256, 8, 4))
        bi = F.HCFused.up(bot, qi, si, x_t, HC, (8, 64, 4))
        for a, b, c in zip(one, two, (di, bot, bi)):
            assert torch.equal(a, b) and torch.equal(a, c), M
        assert not torch.isnan(one[2].float()).any()
        assert int(fx.tickets[:fx._status_at].abs().sum()) == 0
    assert not fx.wait_timeouts()


def test_mix_wait_give_up_then_recovers(gpu, F, monkeypatch):
    """With the flag wait limited to its first read (FP4X_HC_SPIN_LIMIT=0, set
    from the host: every kernel still runs to its end), the workgroups that
    hold no down item give up before the bottleneck is ready: their outputs
    are NaN and the status word is set; the outputs that were computed equal
    the two-launch path.  The call after it waits normally and is
    bit-identical to the two-launch path: the late flag advance of the call
    that gave up cannot satisfy it."""
    rng = np.random.default_rng(78)
    gen = torch.Generator(device=gpu).manual_seed(78)
    qd, sd = F.quantize_w8(torch.randn((336, HC * H), generator=gen, device=gpu) * 0.02)
    qu, su = F.quantize_w8(torch.randn((HC * H, 320), generator=gen, device=gpu) * 0.02)
    qi, si = F.HCFused.interleave_up(qu, su, HC, 8)
    fx = F.HCFused(gpu)
    x_t = bf16_dev(act(rng, 3, HC * H)[0])
    with path_switch(monkeypatch, "FP4X_HC_MIX"):
        ref = fx.mix(x_t, qd, sd, 320, HC, qi, si, x_t, (32, 256, 8, 4))
    assert not fx.wait_timeouts()
    with path_switch(monkeypatch, "FP4X_HC_SPIN_LIMIT", "0"):
        gave_up = fx.mix(x_t, qd, sd, 320, HC, qi, si, x_t, (32, 256, 8, 4))
        torch.cuda.synchronize()
    nan = torch.isnan(gave_up[2].float())
    print(f"give-up call: {int(nan.sum())} of {nan.numel()} block_input values NaN")
    assert nan.any()
    assert torch.equal(gave_up[2][~nan], ref[2][~nan])
    # the down half never gives up: a tile's closer waits only for parts that
    # were dispatched before it and wait on nothing, with at least 65,536 reads
    assert torch.equal(gave_up[0], ref[0]) and torch.equal(gave_up[1], ref[1])
    assert fx.wait_timeouts()
    assert not fx.wait_timeouts()                                                  # cleared by the read
    for _ in range(3):
        again = fx.mix(x_t, qd, sd, 320, HC, qi, si, x_t, (32, 256, 8, 4))
        for a, b in zip(again, ref):
            assert torch.equal(a, b)
        assert int(fx.tickets[:fx._status_at].abs().sum()) == 0
    assert not fx.wait_timeouts()


def took_single_launch(fx):
    """True once a single launch has advanced workgroup 0's generation flag
    (the two-call path never touches the flag lines)."""
    return int(fx.tickets[fx._status_at - 1 + 32].item()) != 0


@pytest.mark.parametrize("h", [1024, 4096])
def test_mix_parts_per_tile(gpu, F, h):
    """The single launch at hidden sizes whose down tiles split into 2 (K = 4096)
    and 8 (K = 16384, the most that keep a tile's parts on one XCD) K parts:
    the tile's last part adds the others' tagged partials in slot order, so
    every call equals the two-launch path bit for bit, with no NaN and no
    status bit."""
    rng = np.random.default_rng(h)
    (qd, sd), (qu, su) = layer(rng, nd=336, lr=320, h=h)
    x, _ = act(rng, 3, HC * h)
    x_t = bf16_dev(x)
    fx = F.HCFused(gpu)
    qd, sd = dev(qd), dev(sd)
    qi, si = F.HCFused.interleave_up(dev(qu), dev(su), HC, 8)
    di, bot = fx.down(x_t, qd, sd, 320, HC, (32, 256, 8, 4))
    bi = F.HCFused.up(bot, qi, si, x_t, HC, (8, 64, 4))
    for _ in range(3):
        one = fx.mix(x_t, qd, sd, 320, HC, qi, si, x_t, (32, 256, 8, 4))
        for a, b in zip(one, (di, bot, bi)):
            assert torch.equal(a, b), h
        assert int(fx.tickets[:fx._status_at].abs().sum()) == 0
    assert took_single_launch(fx), h
    assert not fx.wait_timeouts()


def test_mix_shapes_share_one_buffer(gpu, F):
    """Single launches of different row counts and batch sizes on one scratch
    (so earlier calls leave partials of other layouts where a call keeps its
    own), alternating with the two-launch path: every call equals the
    two-launch result bit for bit, with no NaN and no status bit.  The
    partials' tags come from the call's count, which every call advances in
    every workgroup slot, so no earlier call's partial passes for a later
    one's."""
    rng = np.random.default_rng(515)
    fx = F.HCFused(gpu, n_down=ND, max_ksplit=KS)
    shapes = {}
    for nd, lr, ks in ((ND, LR, KS), (336, 320, 8)):
        (qd, sd), (qu, su) = layer(rng, nd=nd, lr=lr)
        qi, si = F.HCFused.interleave_up(dev(qu), dev(su), HC, 8)
        shapes[nd] = (dev(qd), dev(sd), qi, si, lr, ks)
    for i, (nd, M) in enumerate(((336, 16), (ND, 3), (336, 3), (ND, 1), (336, 1), (ND, 16), (336, 3), (ND, 3))):
        qd, sd, qi, si, lr, ks = shapes[nd]
        x_t = bf16_dev(act(rng, M, HC * H)[0])
        cfg = (32, 256, ks, 4)
        di, bot = fx.down(x_t, qd, sd, lr, HC, cfg)
        bi = F.HCFused.up(bot, qi, si, x_t, HC, (8, 64, 4))
        one = fx.mix(x_t, qd, sd, lr, HC, qi, si, x_t, cfg)
        for a, b in zip(one, (di, bot, bi)):
            assert torch.equal(a, b), (i, nd, M)
        assert int(fx.tickets[:fx._status_at].abs().sum()) == 0
    assert took_single_launch(fx)
    assert not fx.wait_timeouts()


@pytest.mark.parametrize("nd,lr,ks", [(ND, LR, KS), (336, 320, 8)])
def test_mix_late_workgroups(gpu, F, monkeypatch, nd, lr, ks):
    """Workgroups that start after the bottleneck's flag advance.  A kernel on a
    second stream holds most CUs for 4 ms (one workgroup filling a CU's LDS on
    each), and the single-launch mixers issued meanwhile on the current stream
    run on the CUs left free: their up workgroups are dispatched as down items
    end, many after the last down tile has advanced the flags.  Each must find
    its generation reached instead of waiting for another advance: no NaN, no
    status bit, every call bit-identical to the two-launch path.  The flag
    wait is limited to 2^18 reads (tens of ms, set from the host), so a
    workgroup waiting for an advance that never comes ends its call with NaN
    instead of stalling the test."""
    import _fp4x as L
    rng = np.random.default_rng(91 + nd)
    (qd, sd), (qu, su) = layer(rng, nd=nd, lr=lr)
    qd, sd = dev(qd), dev(sd)
    qi, si = F.HCFused.interleave_up(dev(qu), dev(su), HC, 8)
    fx = F.HCFused(gpu, n_down=nd, max_ksplit=ks)
    x_t = bf16_dev(act(rng, 3, HC * H)[0])
    cfg = (32, 256, ks, 4)
    with path_switch(monkeypatch, "FP4X_HC_MIX"):
        ref = fx.mix(x_t, qd, sd, lr, HC, qi, si, x_t, cfg)
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    sink = torch.zeros(1, dtype=torch.int32, device=gpu)
    side = torch.cuda.Stream(gpu)
    with path_switch(monkeypatch, "FP4X_HC_SPIN_LIMIT", str(1 << 18)):
        for free in (cus // 8, cus // 4, cus // 2):
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            L.check(L.lib().fp4x_hold_cus(cus - free, 4000, 160, L.ptr(sink), ctypes.c_void_p(side.cuda_stream)),
                    "hold_cus")
            t0.record()
            outs = [fx.mix(x_t, qd, sd, lr, HC, qi, si, x_t, cfg) for _ in range(8)]
            t1.record()
            torch.cuda.synchronize()
            print(f"{nd}x{HC * H} mixers with {free} of {cus} CUs free: "
                  f"{t0.elapsed_time(t1) * 1e3 / 8:.1f} us per call", flush=True)
            for i, o in enumerate(outs):
                assert not torch.isnan(o[2].float()).any(), (free, i)
                for a, b in zip(o, ref):
                    assert torch.equal(a, b), (free, i)
            assert not fx.wait_timeouts(), free
            assert int(fx.tickets[:fx._status_at].abs().sum()) == 0
    again = fx.mix(x_t, qd, sd, lr, HC, qi, si, x_t, cfg)
    for a, b in zip(again, ref):
        assert torch.equal(a, b)
    assert not fx.wait_timeouts()
