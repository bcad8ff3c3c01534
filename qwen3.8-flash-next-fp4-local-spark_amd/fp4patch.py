"""vLLM general plugin: MI355X decode GEMVs for the FP4-Local hybrid MoE model.

Entry point ``[vllm.general_plugins] fp4x = fp4patch:register`` with the
reference plugin's environment flags and hooks (x/fp4patch.py):

  FP4X_MX8=1        MXFP8 dense linears with M <= FP4X_MX8_MAXM rows read the
                    packed fp8 rows + e8m0 scale rows and run the fp4x GEMV
                    (FP4X_DENSE=mx8|w6|nv4, FP4X_NV4_SHAPES=NxK,...).
  FP4X_HC=1         hyper-connection projections through fp4x GEMVs (M <= 16);
                    FP4X_HC_W8=1 int8 g64 weights, FP4X_HC_FUSED=1 two fused
                    kernels per mixer, FP4X_HC_W8_MTP=1 also the MTP mixers,
                    FP4X_GATE=w8|bf16 router gates, FP4X_MTP_W8=1 MTP linears.
  FP4X_FAST_HEAD=1  target LM head for decode rows: INT2 coarse pass, top-C
                    (FP4X_HEAD_C, default 512) and exact MXFP8 rescore
                    (FP4X_HEAD_G INT2 group size, default 16).

Every install is wrapped so that a failing patch only logs; every hook falls
back to the original method outside its decode shapes.  The kernels are the
HIP kernels of fp4x_kernels (libfp4x.so).
"""
import os
import sys

# (N, K) -> (BN, BK, KSPLIT, warps).  Only KSPLIT (K slices summed in order)
# affects the MI355X kernels; BN/BK/warps are kept for the shape assertion.
CFG_MX8 = {(16384, 2560): (32, 512, 1, 4), (96, 2560): (16, 128, 4, 2), (13312, 2560): (32, 512, 1, 4),
           (640, 2560): (16, 512, 1, 4), (1280, 2560): (16, 512, 1, 4), (2560, 6144): (32, 512, 1, 4),
           (2560, 640): (32, 128, 1, 4)}
CFG_W6 = {(16384, 2560): (32, 256, 1, 4), (96, 2560): (16, 256, 2, 4), (13312, 2560): (32, 256, 1, 4),
          (640, 2560): (16, 256, 1, 4), (1280, 2560): (16, 256, 1, 4), (2560, 6144): (32, 256, 1, 4),
          (2560, 640): (32, 128, 1, 4)}
CFG_NV4 = {}
CFG_BG = {(336, 10240): (16, 512, 4, 4), (10240, 320): (32, 64, 1, 4), (512, 2560): (16, 256, 1, 4)}
CFG_HC_NV4 = {(336, 10240): (16, 128, 2, 4), (10240, 320): (32, 64, 4, 1)}
# The fused mixer's down cfg and the W8 down entry share KSPLIT so that the
# fused and unfused mixers give identical results.
HC_DOWN_CFG = (32, 256, 8, 4)
CFG_W8 = {(336, 10240): (32, 256, 8, 4), (10240, 320): (32, 64, 1, 8), (512, 2560): (16, 512, 1, 4)}
_stats = {"mx8": 0, "mx8_skip": 0}


def _log(msg):
    print(f"[fp4x] {msg}", file=sys.stderr, flush=True)


def _mx8_cfg(n, k):
    c = CFG_MX8.get((n, k))
    if c is None:
        bk = 512 if k % 512 == 0 else 256 if k % 256 == 0 else 128 if k % 128 == 0 else 64
        c = (32, bk, 1, 4)
    return c


def _patch_mx8():
    import torch
    from vllm.model_executor.kernels.linear import b12x_blockscaled as BB
    import fp4x_kernels as F
    maxm = int(os.environ.get("FP4X_MX8_MAXM", "16"))
    dense_mode = os.environ.get("FP4X_DENSE", "mx8")  # mx8 (exact) | w6 | nv4
    nv4_shapes = {tuple(int(v) for v in t.split("x")) for t in os.environ.get("FP4X_NV4_SHAPES", "").split(",") if t}
    qmax = int(os.environ.get("FP4X_DENSE_QMAX", "31"))
    clip = int(os.environ.get("FP4X_DENSE_CLIP", "0"))
    for flag in ("FP4X_DENSE_STATS", "FP4X_DENSE_AWQ"):
        if os.environ.get(flag):
            _log(f"{flag} (activation-aware quality probe) is not part of this build; ignored")
    cache = {}
    orig = BB.B12xBlockscaledLinear.run

    def mode_for(n, k):
        return "nv4" if (n, k) in nv4_shapes else dense_mode

    def lowbit(self, w, s):
        key = id(self)
        q = cache.get(key)
        if q is None and not torch.cuda.is_current_stream_capturing():
            if mode_for(*w.shape) != "w6":
                q = F.requantize_mx8(w, s, "nv4")          # from the packed rows, no fp32 copy
            elif not clip:
                q = F.requantize_mx8(w, s, "w6", qmax=qmax)
            else:                                          # the clip search runs on the torch formulas
                q = F.quantize_w6(F.mx8_dequant(w, s), qmax, clip)
            cache[key] = q
            if len(cache) in (1, 200):
                _log(f"dense {dense_mode}: quantized {len(cache)} layers")
        return q

    seen = set()

    def run(self, source, bias):
        key = (self.recipe, tuple(source.shape), bias is None, getattr(self.packed, "padded_in_features", None),
               getattr(self.packed, "in_features", None))
        if key not in seen and len(seen) < 60:
            seen.add(key)
            _log(f"run {key}")
        if self.recipe == "mxfp8" and source.dim() == 2 and source.shape[0] <= maxm and bias is None:
            pk = self.packed
            w = pk.weight.values
            if w.dtype == torch.uint8:
                w = w.view(torch.float8_e4m3fn)
            if pk.padded_in_features == pk.in_features and w.dtype == torch.float8_e4m3fn and w.dim() == 2:
                s = pk.weight.scale_rows.view(torch.uint8).view(w.shape[0], -1)
                n, k = w.shape
                _stats["mx8"] += 1
                if (_stats["mx8"] + _stats["mx8_skip"]) % 20000 == 0:
                    _log(f"stats {_stats}")
                if dense_mode != "mx8" and n < 100000:
                    q = lowbit(self, w, s)
                    if q is not None:
                        if mode_for(n, k) == "w6":
                            return F.w6_linear(source, *q, CFG_W6.get((n, k)) or (32, 256, 1, 4))
                        return F.nv4_linear(source, *q, CFG_NV4.get((n, k)) or
                                            (32, 256 if k % 256 == 0 else 128 if k % 128 == 0 else 64, 4))
                if os.environ.get("FP4X_MX8_ZERO") == "1":
                    return torch.zeros((source.shape[0], n), dtype=source.dtype, device=source.device)
                return F.mx8_linear(source, w, s, _mx8_cfg(n, k))
        _stats["mx8_skip"] += 1
        if (_stats["mx8"] + _stats["mx8_skip"]) % 20000 == 0:
            _log(f"stats {_stats}")
        return orig(self, source, bias)

    BB.B12xBlockscaledLinear.run = run
    _log(f"MXFP8 decode GEMV installed (M <= {maxm})")


def _patch_hc():
    import torch
    from vllm.models.qwen4_exp.nvidia import hyperconnection as HC
    from vllm.utils.torch_utils import direct_register_custom_op
    import fp4x_kernels as F

    zero = os.environ.get("FP4X_HC_ZERO") == "1"
    w8 = os.environ.get("FP4X_HC_W8") == "1"
    hc_nv4 = os.environ.get("FP4X_HC_NV4") == "1"
    hc_w6 = os.environ.get("FP4X_HC_W6") == "1"
    q4, q6, q8 = {}, {}, {}
    cnt = [0]

    def _quantized(store, w, fn):
        key = (w.data_ptr(), tuple(w.shape))
        qs = store.get(key)
        if qs is None and not torch.cuda.is_current_stream_capturing():
            qs = store[key] = fn(w)
        return qs

    def _bg(x: torch.Tensor, w: torch.Tensor, allow_w8: bool) -> torch.Tensor:
        cnt[0] += 1
        if cnt[0] in (1, 100, 10000):
            _log(f"hc op call #{cnt[0]} x={tuple(x.shape)} w={tuple(w.shape)}")
        small = x.shape[0] <= 16
        if zero and small:
            return torch.zeros((x.shape[0], w.shape[0]), dtype=x.dtype, device=x.device)
        if hc_nv4 and allow_w8 and small:
            qs = _quantized(q4, w, F.quantize_nv4)
            if qs is not None:
                return F.nv4_linear(x.contiguous(), *qs, CFG_HC_NV4.get(tuple(w.shape)) or (32, 64, 4, 1))
        if hc_w6 and allow_w8 and small and tuple(w.shape) != (512, 2560):
            qs = _quantized(q6, w, F.quantize_w6)
            if qs is not None:
                return F.w6_linear(x.contiguous(), *qs, (32, 256 if w.shape[1] % 256 == 0 else 64, 1, 4))
        if w8 and allow_w8 and small:
            qs = _quantized(q8, w, F.quantize_w8)
            if qs is not None:
                if len(q8) in (1, 100):
                    _log(f"HC W8 quantized {len(q8)} weights")
                return F.w8_linear(x.contiguous(), *qs,
                                   CFG_W8.get(tuple(w.shape)) or (32, 256 if w.shape[1] % 256 == 0 else 64, 1, 4))
        if small:
            n, k = w.shape
            return F.bf16_linear(x.contiguous(), w, CFG_BG.get((n, k)) or (32, 256 if k % 256 == 0 else 64, 1, 4))
        return torch.nn.functional.linear(x, w)

    def _bg_fake(x: torch.Tensor, w: torch.Tensor, allow_w8: bool) -> torch.Tensor:
        return x.new_empty((x.shape[0], w.shape[0]))

    direct_register_custom_op(op_name="fp4x_bf16_linear", op_func=_bg, fake_impl=_bg_fake)
    op = torch.ops.vllm.fp4x_bf16_linear
    orig = HC.GatedResidual._mix_normalized
    fused = w8 and os.environ.get("FP4X_HC_FUSED") == "1"
    fx = []
    qu = {}

    def _mix_fused(self, normalized):
        wd = (self.input_mix_weight_down_block_inject if self.use_combine else self.input_mix_weight_down).weight
        wu = self.input_mix_weight_up.weight
        kd, ku = (wd.data_ptr(), tuple(wd.shape)), (wu.data_ptr(), tuple(wu.shape))
        if kd not in q8 or ku not in qu or not fx:
            if torch.cuda.is_current_stream_capturing():
                return None
            if not fx:
                fx.append(F.HCFused(normalized.device, n_down=max(336, wd.shape[0])))
            if kd not in q8:
                q8[kd] = F.quantize_w8(wd)
            if ku not in qu:
                qu[ku] = F.HCFused.interleave_up(*F.quantize_w8(wu), self.hc_count, 8)
                if len(qu) in (1, 97):
                    _log(f"HC fused: prepared {len(qu)} mixers")
        x = normalized.contiguous()
        # HCFused.down then HCFused.up (x/fp4patch.py:217-218), in one launch where the shapes allow
        di, bot, block_input = fx[0].mix(x, *q8[kd], self.lora_rank, self.hc_count, *qu[ku], x, HC_DOWN_CFG,
                                         (8, 64, 4))
        injection = di[:, self.lora_rank: self.lora_rank + self.hc_count] if self.use_combine else None
        return block_input, injection

    def _mix_normalized(self, normalized):
        if self.tp_size > 1:
            return orig(self, normalized)
        aw = "mtp" not in (self._preparation_prefix or "") or os.environ.get("FP4X_HC_W8_MTP") == "1"
        if fused and aw and normalized.shape[0] <= 16:
            r = _mix_fused(self, normalized)
            if r is not None:
                return r
        if self.use_combine:
            down_and_injection = op(normalized, self.input_mix_weight_down_block_inject.weight, aw)
            projected_down = down_and_injection[:, : self.lora_rank]
            injection = down_and_injection[:, self.lora_rank: self.lora_rank + self.hc_count]
        else:
            projected_down = op(normalized, self.input_mix_weight_down.weight, aw)
            injection = None
        small = normalized.shape[0] <= 16 and projected_down.is_cuda
        # The scaled-SiLU and gate-mean epilogues run on the fp4x kernels (the
        # rounding points of the fused mixer) for decode shapes.
        bottleneck = (F.hc_scaled_silu(projected_down, self.lora_rank, self.hc_count) if small
                      else HC.hc_silu(projected_down, self.hc_count))
        gate_logits = op(bottleneck, self.input_mix_weight_up.weight, aw)
        block_input = (F.hc_gate_mean(normalized, gate_logits, self.hc_count) if small
                       else HC.hc_gate_mix(normalized, gate_logits, self.hc_count))
        return block_input, injection

    HC.GatedResidual._mix_normalized = _mix_normalized
    _log("HC decode GEMV installed")
    mtp_w8 = os.environ.get("FP4X_MTP_W8") == "1"
    gate_mode = os.environ.get("FP4X_GATE", "")  # target router gates: w8 | bf16
    if mtp_w8 or gate_mode:
        from vllm.model_executor.layers.linear import UnquantizedLinearMethod
        orig_apply = UnquantizedLinearMethod.apply
        gate_calls = [0]

        def apply(self, layer, x, bias=None):
            if bias is None and layer.weight.dim() == 2:
                prefix = str(getattr(layer, "prefix", ""))
                if mtp_w8 and prefix.startswith("mtp."):
                    x2 = x.reshape(-1, x.shape[-1])
                    return op(x2, layer.weight, True).view(*x.shape[:-1], layer.weight.shape[0])
                if gate_mode and prefix.endswith(".mlp.gate") and x.reshape(-1, x.shape[-1]).shape[0] <= 16:
                    x2 = x.reshape(-1, x.shape[-1]).contiguous()
                    gate_calls[0] += 1
                    if gate_calls[0] in (1, 1000):
                        _log(f"router gate {gate_mode} call #{gate_calls[0]} {prefix} x={tuple(x2.shape)}")
                    if gate_mode == "w8":
                        y = op(x2, layer.weight, True)
                    else:
                        y = F.bf16_linear(x2, layer.weight, CFG_BG.get(tuple(layer.weight.shape)) or (16, 256, 1, 4))
                    return y.view(*x.shape[:-1], layer.weight.shape[0])
            return orig_apply(self, layer, x, bias)

        UnquantizedLinearMethod.apply = apply
        _log(f"UnquantizedLinear decode hook: mtp_w8={mtp_w8} gate={gate_mode or 'off'}")


def _patch_fast_head():
    """Target LM head for decode rows: INT2 coarse pass over the vocabulary,
    top-C candidates per row, exact MXFP8 logits scattered in for them.  The
    argmax is exact whenever the true argmax is among the coarse top-C."""
    import torch
    from vllm.models.qwen4_exp.nvidia import model as MD
    import fp4x_kernels as F
    C = int(os.environ.get("FP4X_HEAD_C", "512"))
    G = int(os.environ.get("FP4X_HEAD_G", "16"))
    orig = MD.Qwen4ExpForCausalLM.compute_logits
    st = {}

    def build(self, h):
        lp = self.logits_processor
        if lp.scale != 1.0 or lp.soft_cap is not None:
            st["off"] = True
            _log("fast head disabled (scale/soft_cap)")
            return
        pk = self.lm_head.b12x_mxfp8_packed_weight
        w = pk.weight.values
        sc = pk.weight.scale_rows.view(torch.uint8).view(w.shape[0], -1)
        st["w"], st["s"] = w, sc
        st["int2"] = os.environ.get("FP4X_HEAD_COARSE", "int2") == "int2"
        # the coarse copy straight from the packed MXFP8 rows (no fp32 copy of the head)
        st["coarse"] = F.requantize_mx8(w, sc, "int2", group=G) if st["int2"] else F.requantize_mx8(w, sc, "nv4")
        ref = orig(self, h)
        st["V"], st["dtype"] = ref.shape[-1], ref.dtype
        out = fast(self, h)
        same = (out.argmax(-1) == ref.argmax(-1)).float().mean().item()
        top = torch.topk(ref.float(), 20, dim=-1).indices
        err = (out.float().gather(1, top) - ref.float().gather(1, top)).abs().max().item()
        _log(f"fast head built: C={C} G={G}; self-check argmax agree {same:.3f}, top20 max|d| {err:.2e}")
        if same < 1.0 or err > 1e-2:
            st["off"] = True
            _log("fast head self-check failed -> disabled")

    def fast(self, h):
        if st["int2"]:
            P, S = st["coarse"]
            # int2_logits + top-C in one call (the coarse kernel also yields the top-k's slice maxima)
            coarse, idx = F.int2_topk(h, P, S, st["w"].shape[0], C)
        else:
            P, S, gs = st["coarse"]
            coarse = F.nv4_linear(h, P, S, gs, (32, 256, 4))
            idx = F.topk_rows(coarse, C)
        return F.refine_mx8_(coarse, h, idx, st["w"], st["s"])

    def compute_logits(self, hidden_states):
        h = hidden_states
        if st.get("off") or h.dim() != 2 or h.shape[0] > 16 or h.shape[0] == 0:
            return orig(self, hidden_states)
        if "coarse" not in st:
            if torch.cuda.is_current_stream_capturing():
                return orig(self, hidden_states)
            build(self, h.contiguous())
            if st.get("off"):
                return orig(self, hidden_states)
        return fast(self, h.contiguous())

    MD.Qwen4ExpForCausalLM.compute_logits = compute_logits
    _log("fast target head patch installed")


# ----------------------------------------------------------------- draft head
# Device scalars 1 / FP4X_DRAFT_TSCALE per device (graph-safe sharpening of the draft logits).
_DRAFT_INV_T = {}


def _draft_prepare(F, w, s, gs, ids, dc, G=16):
    """The MTP draft head's subset of an NVFP4 LM head: rows ids of w [V, K/2]
    and s [V, K/16] (e4m3, row-major), and with dc > 0 their INT2 coarse copy
    (the reference quantizes the fp32 dequant in blocks of 8192 rows; groups are
    row-local, so one pass over the packed rows gives the same codes).
    [x/fp4patch.py:290-307]"""
    st = {"idx": ids, "w": w.index_select(0, ids).contiguous(), "s": s.index_select(0, ids).contiguous(),
          "gs": float(gs)}
    if dc:
        st["c"] = F.requantize_nv4(st["w"], st["s"], st["gs"], "int2", group=G)
    return st


def _draft_logits(F, h, st, vocab, dc, cfg=(32, 256, 4), inv_t=None):
    """Draft logits [M, vocab] bf16: -inf outside the subset.  dc > 0 and M <= 16:
    INT2 coarse over the subset, its top dc (one int2_topk call), their exact
    NVFP4 logits; else the NVFP4 GEMV over the whole subset.  [x/fp4patch.py:309-330]"""
    import torch
    if dc and h.shape[0] <= 16:
        _, cand = F.int2_topk(h, *st["c"], st["idx"].numel(), dc)
        vals = F.refine_nv4(h, cand, st["w"], st["s"], st["gs"])
        return F.scatter_draft(vals, cand, st["idx"], vocab, inv_t)
    sub = F.nv4_linear(h, st["w"], st["s"], st["gs"], cfg)
    full = torch.full((h.shape[0], vocab), float("-inf"), dtype=sub.dtype, device=sub.device)
    full.index_copy_(1, st["idx"], sub)
    return full


def _patch_draft_vocab():
    """MTP draft head over a reduced vocabulary (draft-only; verification stays exact)."""
    import torch
    from vllm.models.qwen4_exp.nvidia import mtp as MTP
    import fp4x_kernels as F
    path = os.environ["FP4X_DRAFT_VOCAB"]
    cfg = tuple(int(v) for v in os.environ.get("FP4X_DRAFT_CFG", "32,256,4").split(","))
    dc = int(os.environ.get("FP4X_DRAFT_INT2", "0"))         # > 0: INT2 coarse + exact rescore of the top dc
    dts = float(os.environ.get("FP4X_DRAFT_TSCALE", "1.0"))  # draft logits / dts
    G = int(os.environ.get("FP4X_DRAFT_INT2_G", "16"))
    orig = MTP.Qwen4ExpMTP.compute_logits

    def build(self, dev):
        lm = self.lm_head
        keep = {int(t) for t in open(path) if t.strip()} | set(range(lm.org_vocab_size - 320, lm.org_vocab_size))
        ids = torch.tensor([i for i in sorted(keep) if i < lm.weight.shape[0]], device=dev, dtype=torch.long)
        sc = lm.weight_scale.data
        n, kb = sc.shape
        # the NVFP4 scale tiles (128 rows x 4 scale columns, stored 32 x 4 x 4) back to row-major
        rows = sc.view(torch.uint8).reshape(n // 128, kb // 4, 32, 4, 4).transpose(1, 3).reshape(n, kb)
        self._fx = _draft_prepare(F, lm.weight.data, rows.view(torch.float8_e4m3fn), lm.weight_global_scale.item(),
                                  ids, dc, G)
        self._fx_vocab = lm.weight.shape[0]
        _log(f"draft vocab head built: {ids.numel()} ids" + (f", INT2 coarse + exact NVFP4 rescore of the top {dc}"
                                                             if dc else ""))

    def compute_logits(self, hidden_states, spec_step_idx=0):
        if getattr(self, "_fx", None) is None:
            if torch.cuda.is_current_stream_capturing() or getattr(self.lm_head, "weight", None) is None:
                return orig(self, hidden_states, spec_step_idx)
            build(self, hidden_states.device)
        h = hidden_states.reshape(-1, hidden_states.shape[-1]).contiguous()
        inv_t = None
        if dts != 1.0:
            if _DRAFT_INV_T.get(h.device) is None:
                _DRAFT_INV_T[h.device] = torch.full((1,), 1.0 / dts, dtype=torch.float32, device=h.device)
            inv_t = _DRAFT_INV_T[h.device]
        return _draft_logits(F, h, self._fx, self._fx_vocab, dc, cfg, inv_t)

    MTP.Qwen4ExpMTP.compute_logits = compute_logits
    _log(f"draft vocab head patch installed ({path})")


# Reference flags whose patches are outside this build (disk PLE embeddings,
# drafter weight swap, MoE ablations, graph debugging).
_NOT_BUILT = ("FP4X_KEEP_GRAPH", "FP4X_MOE_ZERO", "FP4X_MOE_TAU", "FP4X_MTP_PATCH", "FP4X_PLE_SPIN",
              "FP4X_PLE_EARLY", "FP4X_PLE_QD")


def register():
    for flag in _NOT_BUILT:
        if os.environ.get(flag):
            _log(f"{flag} is not part of the MI355X build; ignored")
    if os.environ.get("FP4X_FAST_HEAD") == "1":
        try:
            _patch_fast_head()
        except Exception as e:
            _log(f"fast head patch failed: {type(e).__name__}: {e}")
    if os.environ.get("FP4X_DRAFT_VOCAB"):
        try:
            _patch_draft_vocab()
        except Exception as e:
            _log(f"draft vocab patch failed: {type(e).__name__}: {e}")
    for flag, fn in (("FP4X_MX8", _patch_mx8), ("FP4X_HC", _patch_hc)):
        if os.environ.get(flag) == "1":
            try:
                fn()
            except Exception as e:  # never break serving because of an optional patch
                _log(f"{flag} patch failed: {type(e).__name__}: {e}")
