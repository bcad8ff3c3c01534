"""Stand-ins for the vLLM and b12x classes the fp4x plugin patches, so that
fp4patch.register() and its hooks run without vLLM (which is not installed).

Module paths, class names and the attributes the plugin reads are those of
the reference plugin's targets (x/fp4patch.py:101-139 b12x MXFP8 linear,
:201-249 GatedResidual, :250-275 UnquantizedLinearMethod, :279-333 the MTP
draft head, :337-392 the target LM head).  Each original method is a plain
torch computation that counts its calls, so a hook that falls back to it is
visible.  install() builds fresh classes each time: patches from one test do
not leak into the next.
"""
import sys
import types

import torch


def _mx8_dequant(values, scale_rows):
    w = values.view(torch.float8_e4m3fn).float()
    e = scale_rows.view(torch.uint8).view(w.shape[0], -1).float() - 127.0
    return (w.view(w.shape[0], -1, 32) * torch.exp2(e)[..., None]).view(w.shape)


def _exact_logits(h, wf):
    """bf16(x . w^T) from a float64 sum (the exact dot product, rounded once)."""
    out = torch.empty((h.shape[0], wf.shape[0]), dtype=torch.bfloat16, device=h.device)
    hd = h.double()
    for a in range(0, wf.shape[0], 16384):
        out[:, a:a + 16384] = (hd @ wf[a:a + 16384].double().T).to(torch.float32).to(torch.bfloat16)
    return out


def hc_silu(projected_down, hc_count):
    """bot = bf16(sc * sigmoid(sc)), sc = bf16(float(down) / hc)  (x/fp4x_kernels.py:460-464)."""
    sc = (projected_down.float() / hc_count).to(torch.bfloat16).float()
    return (sc * torch.sigmoid(sc)).to(torch.bfloat16)


def hc_gate_mix(normalized, gate_logits, hc_count):
    """out[m, j] = bf16(sum_s float(bf16(nrm[m, sH + j] * bf16(sigmoid(bf16(g))))) / hc)
    (x/fp4x_kernels.py:486-493); gate_logits rows ordered s * H + j."""
    m = normalized.shape[0]
    g = torch.sigmoid(gate_logits.to(torch.bfloat16).float()).to(torch.bfloat16).float()
    p = (normalized.float() * g).to(torch.bfloat16).float().view(m, hc_count, -1)
    return (p.sum(1) / hc_count).to(torch.bfloat16)


def install():
    """Fresh stand-in modules in sys.modules; returns the classes."""
    names = ["vllm", "vllm.model_executor", "vllm.model_executor.kernels", "vllm.model_executor.kernels.linear",
             "vllm.model_executor.kernels.linear.b12x_blockscaled", "vllm.model_executor.layers",
             "vllm.model_executor.layers.linear", "vllm.models", "vllm.models.qwen4_exp",
             "vllm.models.qwen4_exp.nvidia", "vllm.models.qwen4_exp.nvidia.hyperconnection",
             "vllm.models.qwen4_exp.nvidia.model", "vllm.models.qwen4_exp.nvidia.mtp", "vllm.utils",
             "vllm.utils.torch_utils"]
    mods = {n: types.ModuleType(n) for n in names}
    for n, m in mods.items():
        if "." in n:
            parent, child = n.rsplit(".", 1)
            setattr(mods[parent], child, m)

    class B12xBlockscaledLinear:
        calls = 0

        def __init__(self, values, scale_rows, recipe="mxfp8", padded_in_features=None):
            k = values.shape[1]
            self.recipe = recipe
            self.packed = types.SimpleNamespace(
                weight=types.SimpleNamespace(values=values, scale_rows=scale_rows),
                in_features=k, padded_in_features=k if padded_in_features is None else padded_in_features)

        def run(self, source, bias):
            type(self).calls += 1
            w = _mx8_dequant(self.packed.weight.values, self.packed.weight.scale_rows)
            y = _exact_logits(source, w)
            return y if bias is None else y + bias

    class GatedResidual:
        calls = 0

        def __init__(self, w_down, w_up, lora_rank, hc_count, use_combine=False, prefix="model.layers.0.attn_hc"):
            self.use_combine = use_combine
            if use_combine:
                self.input_mix_weight_down_block_inject = types.SimpleNamespace(weight=w_down)
            else:
                self.input_mix_weight_down = types.SimpleNamespace(weight=w_down)
            self.input_mix_weight_up = types.SimpleNamespace(weight=w_up)
            self.lora_rank, self.hc_count = lora_rank, hc_count
            self.tp_size = 1
            self._preparation_prefix = prefix

        def _mix_normalized(self, normalized):
            type(self).calls += 1
            wd = (self.input_mix_weight_down_block_inject if self.use_combine else self.input_mix_weight_down).weight
            down = (normalized.float() @ wd.float().T).to(torch.bfloat16)
            bot = hc_silu(down[:, :self.lora_rank], self.hc_count)
            gate = (bot.float() @ self.input_mix_weight_up.weight.float().T).to(torch.bfloat16)
            inj = down[:, self.lora_rank:self.lora_rank + self.hc_count] if self.use_combine else None
            return hc_gate_mix(normalized, gate, self.hc_count), inj

    class UnquantizedLinearMethod:
        calls = 0

        def apply(self, layer, x, bias=None):
            type(self).calls += 1
            return torch.nn.functional.linear(x, layer.weight, bias)

    class Qwen4ExpForCausalLM:
        calls = 0

        def __init__(self, values, scale_rows):
            self.logits_processor = types.SimpleNamespace(scale=1.0, soft_cap=None)
            self.lm_head = types.SimpleNamespace(b12x_mxfp8_packed_weight=types.SimpleNamespace(
                weight=types.SimpleNamespace(values=values, scale_rows=scale_rows)))

        def compute_logits(self, hidden_states):
            type(self).calls += 1
            pk = self.lm_head.b12x_mxfp8_packed_weight.weight
            return _exact_logits(hidden_states, _mx8_dequant(pk.values, pk.scale_rows))

    class Qwen4ExpMTP:
        calls = 0

        def __init__(self, weight, weight_scale, global_scale, org_vocab_size):
            self.lm_head = types.SimpleNamespace(weight=weight, weight_scale=weight_scale,
                                                 weight_global_scale=torch.tensor(global_scale),
                                                 org_vocab_size=org_vocab_size)

        def compute_logits(self, hidden_states, spec_step_idx=0):
            type(self).calls += 1
            return None

    def direct_register_custom_op(op_name, op_func, mutates_args=(), fake_impl=None, **kw):
        """torch.ops.vllm.<op_name>: defined once per process (the schema from
        op_func's annotations); a later registration replaces the function."""
        _CURRENT[op_name] = op_func
        if op_name not in _DEFINED:
            lib = torch.library.Library("vllm", "FRAGMENT")
            lib.define(op_name + torch.library.infer_schema(op_func, mutates_args=()))
            lib.impl(op_name, lambda *a: _CURRENT[op_name](*a), "CUDA")
            lib.impl(op_name, lambda *a: _CURRENT[op_name](*a), "CPU")
            _DEFINED[op_name] = lib

    mods["vllm.model_executor.kernels.linear.b12x_blockscaled"].B12xBlockscaledLinear = B12xBlockscaledLinear
    hcm = mods["vllm.models.qwen4_exp.nvidia.hyperconnection"]
    hcm.GatedResidual, hcm.hc_silu, hcm.hc_gate_mix = GatedResidual, hc_silu, hc_gate_mix
    mods["vllm.model_executor.layers.linear"].UnquantizedLinearMethod = UnquantizedLinearMethod
    mods["vllm.models.qwen4_exp.nvidia.model"].Qwen4ExpForCausalLM = Qwen4ExpForCausalLM
    mods["vllm.models.qwen4_exp.nvidia.mtp"].Qwen4ExpMTP = Qwen4ExpMTP
    mods["vllm.utils.torch_utils"].direct_register_custom_op = direct_register_custom_op
    sys.modules.update(mods)
    return types.SimpleNamespace(B12xBlockscaledLinear=B12xBlockscaledLinear, GatedResidual=GatedResidual,
                                 UnquantizedLinearMethod=UnquantizedLinearMethod,
                                 Qwen4ExpForCausalLM=Qwen4ExpForCausalLM, Qwen4ExpMTP=Qwen4ExpMTP)


_DEFINED = {}
_CURRENT = {}


def uninstall():
    for n in [n for n in sys.modules if n == "vllm" or n.startswith("vllm.")]:
        del sys.modules[n]
