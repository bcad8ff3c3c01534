"""The plugin's registration logic on the CPU (x/fp4patch.py:604-647): the
entry point, which FP4X_* switches install which class patches on the
stand-in vLLM modules, the switches the plugin does not implement, and that a patch
that cannot install only logs."""
import os

import pytest

import fake_vllm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen3.8-flash-next-fp4-local-spark_amd")


@pytest.fixture
def plugin(monkeypatch):
    for k in list(os.environ):
        if k.startswith("FP4X_"):
            monkeypatch.delenv(k)
    cls = fake_vllm.install()
    import fp4patch
    yield cls, fp4patch
    fake_vllm.uninstall()


def originals(cls):
    return {"run": cls.B12xBlockscaledLinear.run, "mix": cls.GatedResidual._mix_normalized,
            "apply": cls.UnquantizedLinearMethod.apply, "head": cls.Qwen4ExpForCausalLM.compute_logits,
            "draft": cls.Qwen4ExpMTP.compute_logits}


def test_entry_point():
    text = open(os.path.join(PKG, "fp4patch-0.1.dist-info", "entry_points.txt")).read()
    assert "[vllm.general_plugins]" in text and "fp4x = fp4patch:register" in text


def test_no_switch_no_patch(plugin):
    cls, fp4patch = plugin
    before = originals(cls)
    fp4patch.register()
    assert originals(cls) == before


def test_every_switch_installs_its_hook(plugin, monkeypatch, tmp_path, capfd):
    cls, fp4patch = plugin
    ids = tmp_path / "ids.txt"
    ids.write_text("1\n2\n3\n")
    for k, v in (("FP4X_MX8", "1"), ("FP4X_HC", "1"), ("FP4X_HC_W8", "1"), ("FP4X_GATE", "w8"),
                 ("FP4X_FAST_HEAD", "1"), ("FP4X_DRAFT_VOCAB", str(ids)), ("FP4X_MOE_ZERO", "1")):
        monkeypatch.setenv(k, v)
    before = originals(cls)
    fp4patch.register()
    after = originals(cls)
    assert all(after[k] is not before[k] for k in before), after
    err = capfd.readouterr().err
    for line in ("b12x MXFP8 linears of up to 16 rows", "hyper-connection mixers of up to 16 rows",
                 "unquantized linears hooked", "target LM head of up to 16 rows", "MTP draft head restricted",
                 "FP4X_MOE_ZERO: that reference patch is not implemented by this plugin; ignored"):
        assert line in err, line
    import torch
    assert hasattr(torch.ops.vllm, "fp4x_bf16_linear")            # the plugin's custom op


def test_gate_hook_only_with_its_switches(plugin, monkeypatch):
    cls, fp4patch = plugin
    monkeypatch.setenv("FP4X_HC", "1")
    before = originals(cls)
    fp4patch.register()
    after = originals(cls)
    assert after["mix"] is not before["mix"] and after["apply"] is before["apply"]


def test_failing_patch_only_logs(plugin, monkeypatch, capfd):
    cls, fp4patch = plugin
    import sys
    del sys.modules["vllm.models.qwen4_exp.nvidia.hyperconnection"]
    delattr(sys.modules["vllm.models.qwen4_exp.nvidia"], "hyperconnection")
    monkeypatch.setenv("FP4X_HC", "1")
    monkeypatch.setenv("FP4X_MX8", "1")
    fp4patch.register()                                            # must not raise
    err = capfd.readouterr().err
    assert "FP4X_HC: could not install" in err and "b12x MXFP8 linears" in err


class _FakeScratch:
    """HCFused stand-in: records which launches the hook asks for, and holds a
    status word that poll_timeouts reads and clears."""

    def __init__(self, device, n_down=336):
        self.status, self.calls = 0, []

    def mix(self, x, qd, sd, lr, hc, qi, si, normalized, cfg, up_cfg):
        self.calls.append("mix")
        m = x.shape[0]
        return x.new_zeros((m, qd.shape[0])), x.new_zeros((m, lr)), x.new_zeros((m, qi.shape[0] // hc))

    def down(self, x, qd, sd, lr, hc, cfg):
        self.calls.append("down")
        return x.new_zeros((x.shape[0], qd.shape[0])), x.new_zeros((x.shape[0], lr))

    def poll_timeouts(self):
        hit, self.status = bool(self.status & 1), 0
        return hit


def _fake_kernels():
    import types
    F = types.ModuleType("fp4x_kernels")
    made = []

    class HCFused(_FakeScratch):
        def __init__(self, device, n_down=336):
            super().__init__(device, n_down)
            made.append(self)

        @staticmethod
        def interleave_up(q, s, hc, bj):
            return q, s

        @staticmethod
        def up(bot, qi, si, normalized, hc, cfg):
            made[0].calls.append("up")
            return bot.new_zeros((bot.shape[0], qi.shape[0] // hc))

    F.HCFused, F.made = HCFused, made
    F.quantize_w8 = lambda w: (w, w)
    return F


def test_mixer_timeout_switches_to_two_launches(plugin, monkeypatch, capfd):
    """A single-launch mixer whose wait gave up sets the status word; the hook's
    next status check (from an eager fast-head call, or every CHECK_EVERY-th
    eager mixer call) logs and counts it, and the fused mixers then run as two
    launches (down, then up)."""
    import sys
    import torch
    cls, fp4patch = plugin
    F = _fake_kernels()
    monkeypatch.setitem(sys.modules, "fp4x_kernels", F)
    monkeypatch.setattr(fp4patch, "_capturing", lambda torch_mod: False)
    monkeypatch.setattr(fp4patch, "MIXERS", [])
    for k in ("FP4X_HC", "FP4X_HC_W8", "FP4X_HC_FUSED"):
        monkeypatch.setenv(k, "1")
    fp4patch.register()
    assert len(fp4patch.MIXERS) == 1
    mixer = fp4patch.MIXERS[0]
    hc, h, lr = 4, 64, 16
    res = cls.GatedResidual(torch.zeros((24, hc * h)), torch.zeros((hc * h, lr)), lr, hc)
    x = torch.zeros((3, hc * h), dtype=torch.bfloat16)
    res._mix_normalized(x)
    fx = F.made[0]
    assert fx.calls == ["mix"] and cls.GatedResidual.calls == 0
    mixer.check_waits()                                    # nothing set: stays single-launch
    res._mix_normalized(x)
    assert fx.calls[-1] == "mix"
    fx.status = 1                                          # a call gave up
    res._mix_normalized(x)
    assert fx.calls[-1] == "mix"                           # not seen until a check
    head = cls.Qwen4ExpForCausalLM(torch.zeros((8, 32), dtype=torch.uint8), torch.zeros((8, 1), dtype=torch.uint8))
    monkeypatch.setenv("FP4X_FAST_HEAD", "1")
    for k in ("FP4X_HC", "FP4X_HC_W8", "FP4X_HC_FUSED"):
        monkeypatch.delenv(k)
    fp4patch.register()                                    # the fast head: its eager calls check the mixers
    head.compute_logits(torch.zeros((20, 32), dtype=torch.bfloat16))   # 20 rows: the original head runs
    assert mixer.timeouts == 1 and not mixer.single and fx.status == 0
    assert "gave up waiting for its bottleneck" in capfd.readouterr().err
    n = len(fx.calls)
    res._mix_normalized(x)
    assert fx.calls[n:] == ["down", "up"]
    # the periodic check from the mixer's own eager calls
    mixer.single, fx.status = True, 1
    for _ in range(mixer.CHECK_EVERY):
        res._mix_normalized(x)
    assert mixer.timeouts == 2 and not mixer.single
    assert fp4patch.STATS.n.get("mix_timeout", 0) >= 2


def test_periodic_stats(plugin, capfd):
    """The hooks' call counts are logged every `every` counted calls."""
    cls, fp4patch = plugin
    st = fp4patch._Stats(every=3)
    for key in ("mx8", "mx8_skip", "mx8", "mx8"):
        st.count(key)
    err = capfd.readouterr().err
    assert "stats {'mx8': 2, 'mx8_skip': 1}" in err and err.count("stats") == 1
