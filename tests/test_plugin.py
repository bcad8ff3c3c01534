"""The plugin's registration logic on the CPU (x/fp4patch.py:604-647): the
entry point, which FP4X_* switches install which class patches on the
stand-in vLLM modules, the switches outside this build, and that a patch
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
                 "FP4X_MOE_ZERO: that reference patch is not part of this build; ignored"):
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
