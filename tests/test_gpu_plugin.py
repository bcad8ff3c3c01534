"""The plugin boundary (x/fp4patch.py): register() under each FP4X_* switch
patches the stand-in vLLM classes of tests/fake_vllm.py; the patched methods
run the HIP kernels on decode shapes, with results equal bit for bit to the
direct fp4x_kernels calls the hooks stand for, and fall back to the original
methods outside those shapes."""
import os

import numpy as np
import pytest
import torch

import fake_vllm

pytestmark = pytest.mark.gpu


@pytest.fixture
def plugin(monkeypatch):
    for k in list(os.environ):
        if k.startswith("FP4X_"):
            monkeypatch.delenv(k)
    cls = fake_vllm.install()
    import fp4patch
    import fp4x_kernels
    fp4patch._DRAFT_INV_T.clear()
    yield cls, fp4patch, fp4x_kernels
    fake_vllm.uninstall()


def bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


def test_dense_mx8_hook(gpu, plugin, monkeypatch):
    """FP4X_MX8=1: b12x's MXFP8 run() goes to mx8_linear for M <= 16 rows, no
    bias and unpadded K (x/fp4patch.py:101-137); other calls keep the original."""
    cls, fp4patch, F = plugin
    monkeypatch.setenv("FP4X_MX8", "1")
    fp4patch.register()
    g = torch.Generator(device=gpu).manual_seed(1)
    q, s = F.quantize_mx8(torch.randn((4096, 2560), generator=g, device=gpu) * 0.02)
    lin = cls.B12xBlockscaledLinear(q, s)
    for m in (1, 3, 16):
        x = torch.randn((m, 2560), generator=g, device=gpu).to(torch.bfloat16)
        want = F.mx8_linear(x, q.view(torch.float8_e4m3fn), s, fp4patch._mx8_cfg(4096, 2560))
        assert torch.equal(bits(lin.run(x, None)), bits(want))
    assert cls.B12xBlockscaledLinear.calls == 0
    x = torch.randn((3, 2560), generator=g, device=gpu).to(torch.bfloat16)
    lin.run(x, torch.zeros(4096, dtype=torch.bfloat16, device=gpu))                      # bias
    lin.run(torch.randn((17, 2560), generator=g, device=gpu).to(torch.bfloat16), None)   # M > FP4X_MX8_MAXM
    cls.B12xBlockscaledLinear(q, s, recipe="nvfp4").run(x, None)                          # another recipe
    cls.B12xBlockscaledLinear(q, s, padded_in_features=2688).run(x, None)                 # padded K
    assert cls.B12xBlockscaledLinear.calls == 4


@pytest.mark.parametrize("mode", ["w6", "nv4"])
def test_dense_lowbit_hook(gpu, plugin, monkeypatch, mode):
    """FP4X_DENSE=w6|nv4: the MXFP8 weights are requantized once per layer from
    their fp32 dequant and served by w6_linear / nv4_linear."""
    cls, fp4patch, F = plugin
    monkeypatch.setenv("FP4X_MX8", "1")
    monkeypatch.setenv("FP4X_DENSE", mode)
    fp4patch.register()
    g = torch.Generator(device=gpu).manual_seed(2)
    q, s = F.quantize_mx8(torch.randn((8192, 2560), generator=g, device=gpu) * 0.02)
    lin = cls.B12xBlockscaledLinear(q, s)
    x = torch.randn((3, 2560), generator=g, device=gpu).to(torch.bfloat16)
    got = lin.run(x, None)
    wf = F.mx8_dequant(q.view(torch.float8_e4m3fn), s)
    if mode == "w6":
        want = F.w6_linear(x, *F.quantize_w6(wf), fp4patch.CFG_W6.get((8192, 2560)) or (32, 256, 1, 4))
    else:
        want = F.nv4_linear(x, *F.quantize_nv4(wf), (32, 256, 4))
    assert torch.equal(bits(got), bits(want))
    assert torch.equal(bits(lin.run(x, None)), bits(want))                  # the cached weights
    assert cls.B12xBlockscaledLinear.calls == 0


def _mixer(gpu, seed, lr=320, hc=4, H=2560):
    g = torch.Generator(device=gpu).manual_seed(seed)
    wd = (torch.randn((336, hc * H), generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    wu = (torch.randn((hc * H, lr), generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    x = torch.randn((3, hc * H), generator=g, device=gpu).to(torch.bfloat16)
    return wd, wu, x


def test_mixer_fused_equals_unfused(gpu, plugin, monkeypatch):
    """FP4X_HC=1 FP4X_HC_W8=1: the fused mixer (FP4X_HC_FUSED=1, HCFused.mix)
    and the unfused W8 path through the registered custom op give identical
    block input and injection (x/fp4patch.py:201-249)."""
    cls, fp4patch, F = plugin
    wd, wu, x = _mixer(gpu, 3)
    monkeypatch.setenv("FP4X_HC", "1")
    monkeypatch.setenv("FP4X_HC_W8", "1")
    monkeypatch.setenv("FP4X_HC_FUSED", "1")
    fp4patch.register()
    res = cls.GatedResidual(wd, wu, 320, 4, use_combine=True)
    bi_f, inj_f = res._mix_normalized(x)
    bi_f2, _ = res._mix_normalized(x)                                   # prepared weights reused
    monkeypatch.delenv("FP4X_HC_FUSED")
    cls = fake_vllm.install()
    fp4patch.register()
    res = cls.GatedResidual(wd, wu, 320, 4, use_combine=True)
    bi_u, inj_u = res._mix_normalized(x)
    assert cls.GatedResidual.calls == 0
    assert bi_f.shape == (3, 2560) and inj_f.shape == (3, 4)
    assert torch.equal(bits(bi_f), bits(bi_u)) and torch.equal(bits(inj_f), bits(inj_u))
    assert torch.equal(bits(bi_f), bits(bi_f2))
    # the unfused path is the documented composition of the kernels
    q, s = F.quantize_w8(wd)
    down = F.w8_linear(x, q, s, fp4patch.CFG_W8[(336, 10240)])
    bot = F.hc_scaled_silu(down[:, :320], 320, 4)
    qu, su = F.quantize_w8(wu)
    gate = F.w8_linear(bot, qu, su, fp4patch.CFG_W8[(10240, 320)])
    assert torch.equal(bits(bi_u), bits(F.hc_gate_mean(x, gate, 4)))
    assert torch.equal(bits(inj_u), bits(down[:, 320:324]))


def test_mixer_mtp_and_large_batches(gpu, plugin, monkeypatch):
    """MTP mixers take the bf16 GEMVs unless FP4X_HC_W8_MTP=1; more than 16
    rows take torch's linear and the model's own epilogues."""
    cls, fp4patch, F = plugin
    wd, wu, x = _mixer(gpu, 4)
    for k in ("FP4X_HC", "FP4X_HC_W8", "FP4X_HC_FUSED"):
        monkeypatch.setenv(k, "1")
    fp4patch.register()
    wd = wd[:320].contiguous()                        # without the injection rows: [lora_rank, K]
    res = cls.GatedResidual(wd, wu, 320, 4, prefix="mtp.layers.0.attn_hc")
    bi, inj = res._mix_normalized(x)
    assert inj is None
    down = F.bf16_linear(x, wd, (32, 256, 1, 4))
    bot = F.hc_scaled_silu(down, 320, 4)
    gate = F.bf16_linear(bot, wu, fp4patch.CFG_BG[(10240, 320)])
    assert torch.equal(bits(bi), bits(F.hc_gate_mean(x, gate, 4)))
    big = torch.randn((20, 10240), device=gpu).to(torch.bfloat16)
    bi20, _ = cls.GatedResidual(wd, wu, 320, 4)._mix_normalized(big)
    assert bi20.shape == (20, 2560) and bool(torch.isfinite(bi20.float()).all())
    assert cls.GatedResidual.calls == 0


@pytest.mark.parametrize("mode", ["w8", "bf16"])
def test_router_gate_and_mtp_linear_hooks(gpu, plugin, monkeypatch, mode):
    """FP4X_GATE=w8|bf16 routes `*.mlp.gate` linears of at most 16 rows, and
    FP4X_MTP_W8=1 the `mtp.*` linears, through the fp4x GEMVs
    (x/fp4patch.py:250-275); other linears keep the original method."""
    cls, fp4patch, F = plugin
    for k, v in (("FP4X_HC", "1"), ("FP4X_HC_W8", "1"), ("FP4X_GATE", mode), ("FP4X_MTP_W8", "1")):
        monkeypatch.setenv(k, v)
    fp4patch.register()
    g = torch.Generator(device=gpu).manual_seed(5)
    W = (torch.randn((512, 2560), generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    x = torch.randn((3, 2560), generator=g, device=gpu).to(torch.bfloat16)
    meth = cls.UnquantizedLinearMethod()
    gate = type("L", (), {})()
    gate.weight, gate.prefix = W, "model.layers.7.mlp.gate"
    y = meth.apply(gate, x)
    if mode == "w8":
        want = F.w8_linear(x, *F.quantize_w8(W), fp4patch.CFG_W8[(512, 2560)])
    else:
        want = F.bf16_linear(x, W, fp4patch.CFG_BG[(512, 2560)])
    assert torch.equal(bits(y), bits(want))
    mtp = type("L", (), {})()
    mtp.weight, mtp.prefix = (torch.randn((1280, 2560), generator=g, device=gpu) * 0.02).to(torch.bfloat16), "mtp.fc"
    y = meth.apply(mtp, x.view(1, 3, 2560))
    assert y.shape == (1, 3, 1280)
    assert torch.equal(bits(y[0]), bits(F.w8_linear(x, *F.quantize_w8(mtp.weight), (32, 256, 1, 4))))
    other = type("L", (), {})()
    other.weight, other.prefix = W, "model.layers.7.mlp.experts"
    meth.apply(other, x)
    assert cls.UnquantizedLinearMethod.calls == 1


def _head(F, gpu, V, K, on_grid):
    """MXFP8 head rows: N(0, 0.02), or rows on the INT2 grid ((c - 1.5) * 2^-8,
    64 rows at 2^-4, every 16-group holding a code of magnitude 1.5), which
    INT2 and MXFP8 both hold exactly, so coarse and exact logits agree."""
    g = torch.Generator(device=gpu).manual_seed(6)
    if on_grid:
        c = torch.randint(0, 4, (V, K), generator=g, device=gpu)
        c[:, ::16] = torch.randint(0, 2, (V, K // 16), generator=g, device=gpu) * 3
        sc = torch.full((V, 1), 2.0 ** -8, device=gpu)
        sc[torch.randperm(V, generator=g, device=gpu)[:64]] = 2.0 ** -4
        w = (c.float() - 1.5) * sc
    else:
        w = torch.randn((V, K), generator=g, device=gpu) * 0.02
    q, s = F.quantize_mx8(w)
    assert not on_grid or torch.equal(F.mx8_dequant(q.view(torch.float8_e4m3fn), s), w)
    return q, s, torch.randn((3, K), generator=g, device=gpu).to(torch.bfloat16)


def test_fast_head_hook(gpu, plugin, monkeypatch):
    """FP4X_FAST_HEAD=1 on rows INT2 holds exactly: the first eager call
    builds the INT2 copy and passes the reference's self-check against the
    original head (x/fp4patch.py:349-368); every call returns coarse logits
    with the top-512 rows' exact MXFP8 logits scattered in, the original's
    argmax, and the original's values on its top 20.  M > 16 keeps the original."""
    cls, fp4patch, F = plugin
    monkeypatch.setenv("FP4X_FAST_HEAD", "1")
    fp4patch.register()
    V, K = 65536 + 128, 2560
    q, s, h = _head(F, gpu, V, K, True)
    head = cls.Qwen4ExpForCausalLM(q.view(torch.float8_e4m3fn), s)
    first = head.compute_logits(h)
    assert cls.Qwen4ExpForCausalLM.calls == 1                           # the self-check's reference call
    out = head.compute_logits(h)
    assert cls.Qwen4ExpForCausalLM.calls == 1
    assert torch.equal(bits(first), bits(out))
    exact = fake_vllm._exact_logits(h, fake_vllm._mx8_dequant(q, s))
    assert torch.equal(out.argmax(-1), exact.argmax(-1))
    top = torch.topk(exact.float(), 20, dim=-1).indices
    assert float((out.float().gather(1, top) - exact.float().gather(1, top)).abs().max()) <= 1e-2
    # the other entries: the coarse INT2 logits, the top 512 of them rescored in place
    coarse = F.int2_logits(h, *F.quantize_int2(F.mx8_dequant(q.view(torch.float8_e4m3fn), s), group=16), V,
                           out_dtype=torch.bfloat16)
    idx = F.topk_rows(coarse, 512)
    keep = torch.ones_like(coarse, dtype=torch.bool).scatter_(1, idx, False)
    assert torch.equal(bits(out)[keep], bits(coarse)[keep])
    d = (out.float().gather(1, idx) - exact.float().gather(1, idx)).abs()
    ulp = exact.float().gather(1, idx).abs().clamp_min(2.0 ** -126) * 2.0 ** -7
    assert bool((d <= ulp).all())                                       # exact logits, one bf16 rounding apart
    assert head.compute_logits(torch.randn((17, K), device=gpu).to(torch.bfloat16)).shape == (17, V)
    assert cls.Qwen4ExpForCausalLM.calls == 2                           # M > 16: the original


def test_fast_head_self_check_disables(gpu, plugin, monkeypatch):
    """When the original head disagrees with the fast copy (here: +4 on one
    column) the self-check fails and every call keeps the original head; a
    logits processor with a scale or soft cap turns the hook off unbuilt."""
    cls, fp4patch, F = plugin
    base = cls.Qwen4ExpForCausalLM.compute_logits

    def skewed(self, h):
        out = base(self, h)
        out[:, 5] += 4
        return out

    cls.Qwen4ExpForCausalLM.compute_logits = skewed
    monkeypatch.setenv("FP4X_FAST_HEAD", "1")
    fp4patch.register()
    q, s, h = _head(F, gpu, 65536 + 128, 2560, True)
    head = cls.Qwen4ExpForCausalLM(q.view(torch.float8_e4m3fn), s)
    a = head.compute_logits(h)
    b = head.compute_logits(h)
    assert cls.Qwen4ExpForCausalLM.calls == 3                           # self-check, then the original twice
    assert torch.equal(bits(a), bits(b))
    cls = fake_vllm.install()
    fp4patch.register()
    head = cls.Qwen4ExpForCausalLM(q.view(torch.float8_e4m3fn), s)
    head.logits_processor.scale = 0.5
    head.compute_logits(h)
    head.compute_logits(h)
    assert cls.Qwen4ExpForCausalLM.calls == 2


def _swizzle(rows):
    """Row-major [n, kb] NVFP4 scales -> the b12x tile layout the plugin undoes
    (x/fp4patch.py:296): tiles of 128 rows x 4 columns stored 32 x 4 x 4."""
    n, kb = rows.shape
    return rows.reshape(n // 128, 4, 32, kb // 4, 4).transpose(1, 3).contiguous().reshape(n, kb)


@pytest.mark.parametrize("dc,tscale", [(64, "1.0"), (64, "0.8"), (0, "1.0")])
def test_draft_vocab_hook(gpu, plugin, monkeypatch, tmp_path, dc, tscale):
    """FP4X_DRAFT_VOCAB: the MTP head serves the listed ids plus the last 320
    of the vocabulary from its NVFP4 rows, after undoing b12x's scale tiles;
    dc > 0 takes the INT2 + top-dc + exact rescore path, FP4X_DRAFT_TSCALE
    divides the rescored logits (x/fp4patch.py:279-334)."""
    cls, fp4patch, F = plugin
    V, K, M = 235 * 128, 2560, 3
    rng = np.random.default_rng(7)
    listed = rng.choice(V - 320, 6000, replace=False)
    path = tmp_path / "ids.txt"
    path.write_text("\n".join(str(int(i)) for i in listed) + "\n\n")
    monkeypatch.setenv("FP4X_DRAFT_VOCAB", str(path))
    monkeypatch.setenv("FP4X_DRAFT_INT2", str(dc))
    monkeypatch.setenv("FP4X_DRAFT_TSCALE", tscale)
    fp4patch.register()
    g = torch.Generator(device=gpu).manual_seed(8)
    P, S, gs = F.quantize_nv4(torch.randn((V, K), generator=g, device=gpu) * 0.02)
    mtp = cls.Qwen4ExpMTP(P, _swizzle(S.view(torch.uint8)).view(torch.float8_e4m3fn), gs, V)
    h = torch.randn((1, M, K), generator=g, device=gpu).to(torch.bfloat16)
    got = mtp.compute_logits(h)
    assert cls.Qwen4ExpMTP.calls == 0 and got.shape == (M, V)
    ids = torch.tensor(sorted(set(int(i) for i in listed) | set(range(V - 320, V))), device=gpu)
    st = fp4patch._draft_prepare(F, P, S, gs, ids, dc)
    inv_t = None if tscale == "1.0" else torch.full((1,), 1.0 / float(tscale), device=gpu)
    want = fp4patch._draft_logits(F, h.view(M, K), st, V, dc, (32, 256, 4), inv_t)
    assert torch.equal(bits(got), bits(want))
    outside = torch.ones(V, dtype=torch.bool, device=gpu)
    outside[ids] = False
    assert bool((bits(got)[:, outside] == -128).all())                  # bf16 -inf
