"""GPU parity of the hyper-connection mixer kernels.

* fused (hc_down + hc_up) and unfused (W8 GEMV, scaled SiLU, W8 GEMV, gate
  mean) agree bit for bit, over 97 seeded layers at the synthetic shape
  (x [3, 4 x 2560], W_down [640, 10240], W_up [10240, 640], 16 K-splits);
* both match the oracle: DI within the MFMA accumulation bound of the exact
  sum plus bf16 rounding, block_input within bf16 rounding of the oracle's
  float64-sigmoid epilogue;
* the split-K scratch is re-armed: tickets are zero after every call;
* the whole mixer in one call (HCFused.mix, one launch where the shapes allow)
  equals down + up bit for bit and re-arms its counters.
"""
import numpy as np
import pytest
import torch

from oracle import formats as fm
from oracle import hc as ohc
from oracle import ordered
from oracle import quant as oq

from gpu_helpers import act, assert_tol, bf16_bits, bf16_dev, dev, to_f32

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
    return di, bot, F.hc_gate_mean(x_t, g, HC)


def test_fused_equals_unfused_97_layers(gpu, F):
    rng = np.random.default_rng(2024)
    gen = torch.Generator(device=gpu).manual_seed(2024)
    fx = F.HCFused(gpu, n_down=ND, max_ksplit=KS)
    x, xb = act(rng, 3, HC * H)
    x_t = bf16_dev(x)
    worst = 0.0
    for i in range(97):
        wd = torch.randn((ND, HC * H), generator=gen, device=gpu) * 0.02
        wu = torch.randn((HC * H, LR), generator=gen, device=gpu) * 0.02
        qd_t, sd_t = F.quantize_w8(wd)
        qu_t, su_t = F.quantize_w8(wu)
        qi, si = F.HCFused.interleave_up(qu_t, su_t, HC, 8)
        di, bot = fx.down(x_t, qd_t, sd_t, LR, HC, (32, 256, KS, 4))
        bi = F.HCFused.up(bot, qi, si, x_t, HC, (8, 64, 4))
        di2, bot2, bi2 = unfused(F, x_t, qd_t, sd_t, qu_t, su_t, LR, KS)
        assert torch.equal(di, di2) and torch.equal(bot, bot2) and torch.equal(bi, bi2), f"layer {i}"
        assert int(fx.tickets.abs().sum()) == 0
        di3, bot3, bi3 = fx.mix(x_t, qd_t, sd_t, LR, HC, qi, si, x_t, (32, 256, KS, 4))
        assert torch.equal(di, di3) and torch.equal(bot, bot3) and torch.equal(bi, bi3), f"layer {i} mix"
        assert int(fx.tickets.abs().sum()) == 0
        if i % 24 == 0:
            import _fp4x
            qd, sd, qu, su = (t.cpu().numpy() for t in (qd_t, sd_t, qu_t, su_t))
            lpr, _ = _fp4x.layout(_fp4x.FMT_W8_F32, HC * H // KS)
            wop = fm.round_bf16(oq.dequant_w8(qd, sd))
            exact = ordered.exact_sum(x, wop)
            bound = ordered.mfma_bound(x, wop, KS) + np.abs(exact) * 2.0 ** -8
            assert np.all(np.abs(to_f32(di) - exact) <= bound), f"layer {i} down"
            _, _, bi_ref = ohc.mixer(x, qd, sd, qu, su, LR, HC)
            bot_o = ohc.scaled_silu(to_f32(di)[:, :LR], HC)       # the epilogue alone, from the GPU's di
            assert np.abs(to_f32(bot) - bot_o).max() <= np.abs(bot_o).max() * 2 ** -7
            assert_tol(to_f32(bi), bi_ref, rel=2e-2, abs_=2e-2, what=f"layer {i} block_input")
            worst = max(worst, float(np.abs(to_f32(bi) - bi_ref).max()))
    print(f"block_input max |d| vs oracle over sampled layers: {worst:.3g}")


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
    di2, bot2, bi2 = unfused(F, x_t, dev(qd), dev(sd), dev(qu), dev(su), 320, 8)
    assert torch.equal(di, di2) and torch.equal(bot, bot2) and torch.equal(bi, bi2)
    for _ in range(3):                                # one launch, counters re-armed every call
        di3, bot3, bi3 = fx.mix(x_t, dev(qd), dev(sd), 320, HC, qi, si, x_t, (32, 256, 8, 4))
        assert torch.equal(di, di3) and torch.equal(bot, bot3) and torch.equal(bi, bi3)
        assert int(fx.tickets.abs().sum()) == 0
    di_ref, _, bi_ref = ohc.mixer(x, qd, sd, qu, su, 320, HC)
    assert_tol(to_f32(di), di_ref, what="di")
    assert_tol(to_f32(bi), bi_ref, rel=2e-2, abs_=2e-2, what="block_input")


def test_epilogue_kernels_vs_oracle(gpu, F):
    rng = np.random.default_rng(3)
    d = fm.round_bf16((rng.standard_normal((3, 700)) * 4).astype(np.float32))
    bot = F.hc_scaled_silu(bf16_dev(d), 640, HC)
    ref = ohc.scaled_silu(d[:, :640], HC)
    assert np.abs(to_f32(bot) - ref).max() <= 2 ** -7 * np.abs(ref).max()
    assert (bf16_bits(bot) == fm.bf16_bits(ref)).mean() > 0.99
    nrm = fm.round_bf16(rng.standard_normal((3, HC * 64)).astype(np.float32))
    g = fm.round_bf16((rng.standard_normal((3, HC * 64)) * 3).astype(np.float32))
    out = F.hc_gate_mean(bf16_dev(nrm), bf16_dev(g), HC)
    ref = ohc.gate_mean(nrm, g, HC)
    assert (bf16_bits(out) == fm.bf16_bits(ref)).mean() > 0.99
    assert_tol(to_f32(out), ref, rel=1e-2, abs_=1e-2, what="gate_mean")


def test_mix_fallback_and_fp16_scales(gpu, F, monkeypatch):
    """The two-call fallback (FP4X_HC_MIX=0) and the single launch agree, with
    fp16 scales, across repeated calls sharing one scratch."""
    rng = np.random.default_rng(77)
    gen = torch.Generator(device=gpu).manual_seed(77)
    wd = torch.randn((336, HC * H), generator=gen, device=gpu) * 0.02
    wu = torch.randn((HC * H, 320), generator=gen, device=gpu) * 0.02

    def f16(w):
        g = w.reshape(w.shape[0], -1, 64)
        s16 = (g.abs().amax(-1).clamp_min(1e-12) / 127.0).half()
        q = torch.round(g / s16.float().unsqueeze(-1)).clamp(-127, 127).to(torch.int8).reshape(w.shape)
        return q.contiguous(), s16.contiguous()

    qd, sd = f16(wd)
    qu, su = f16(wu)
    qi, si = F.HCFused.interleave_up(qu, su, HC, 8)
    fx = F.HCFused(gpu)
    for M in (3, 16, 1):
        x_t = bf16_dev(act(rng, M, HC * H)[0])
        one = fx.mix(x_t, qd, sd, 320, HC, qi, si, x_t, (32, 256, 8, 4))
        monkeypatch.setenv("FP4X_HC_MIX", "0")
        two = fx.mix(x_t, qd, sd, 320, HC, qi, si, x_t, (32, 256, 8, 4))
        monkeypatch.delenv("FP4X_HC_MIX")
        di, bot = fx.down(x_t, qd, sd, 320, HC, (32, 256, 8, 4))
        bi = F.HCFused.up(bot, qi, si, x_t, HC, (8, 64, 4))
        for a, b, c in zip(one, two, (di, bot, bi)):
            assert torch.equal(a, b) and torch.equal(a, c), M
        assert not torch.isnan(one[2].float()).any()
        assert int(fx.tickets.abs().sum()) == 0
