"""vLLM general plugin routing the decode-shaped GEMVs of the FP4-Local hybrid
MoE model to the MI355X kernels of fp4x_kernels (libfp4x.so).

Entry point ``[vllm.general_plugins] fp4x = fp4patch:register``.  The
switches, the classes patched, the shapes each hook takes and the fallbacks
are those of the reference plugin (x/fp4patch.py), which is the drop-in
contract:

  FP4X_MX8=1        b12x MXFP8 linears with at most FP4X_MX8_MAXM rows:
                    FP4X_DENSE=mx8 (the packed rows as they are) | w6 | nv4
                    (a low-bit copy made once per layer), FP4X_NV4_SHAPES
                    lists NxK shapes that take NVFP4 under FP4X_DENSE=w6.
  FP4X_HC=1         hyper-connection projections of at most 16 rows through
                    the custom op vllm::fp4x_bf16_linear: FP4X_HC_W8=1 int8
                    g64 copies, FP4X_HC_FUSED=1 the whole mixer in one call,
                    FP4X_HC_W8_MTP=1 also for the MTP layers' mixers,
                    FP4X_GATE=w8|bf16 the router gates, FP4X_MTP_W8=1 the
                    MTP layers' linears.
  FP4X_FAST_HEAD=1  target LM head of at most 16 rows: INT2 coarse logits
                    (FP4X_HEAD_G group size), their top FP4X_HEAD_C rows
                    rescored exactly from the MXFP8 head.
  FP4X_DRAFT_VOCAB  MTP draft head restricted to the token ids of a file
                    (FP4X_DRAFT_INT2 > 0: INT2 coarse + exact NVFP4 rescore
                    of the top FP4X_DRAFT_INT2 ids; FP4X_DRAFT_TSCALE).

A patch that cannot install is reported and skipped, and every hook hands
calls outside its shapes (and calls met during graph capture before its
weights are prepared) back to the method it replaced.
"""
import os
import sys

# Tile tables keyed by weight shape (N, K): (BN, BK, KSPLIT, warps), or
# (BN, BK, warps, KSPLIT) for NVFP4.  The MI355X kernels choose their own
# tiling; KSPLIT (how many K slices are summed, in order) and the shape
# assertion on (K, KSPLIT, BK) are what these entries still decide.  The values
# are the reference's (x/fp4patch.py:11-21) except two K splits:
#   * CFG_W8[(336, 10240)] sums 8 K slices (the reference: 4) so that the
#     unfused mixer's down projection takes the fused one's decomposition
#     (HC_DOWN_CFG) and the two paths give the same bits;
#   * CFG_BG[(336, 10240)] sums 4 K slices (the reference: 1).  With one slice
#     this 21-tile bf16 GEMV has 21 workgroups for 256 CUs; four ordered slices
#     spread it over 84, and fix its summation order as any split does.  (On
#     the reference's GPU the same table entry takes one slice because its
#     split-K adds partials with fp32 atomics in no fixed order.)
CFG_MX8 = {(16384, 2560): (16, 512, 1, 4), (96, 2560): (16, 128, 4, 2), (13312, 2560): (32, 512, 1, 4),
           (640, 2560): (16, 512, 1, 2), (1280, 2560): (16, 256, 1, 4), (2560, 6144): (32, 512, 1, 4),
           (2560, 640): (64, 128, 1, 4)}
CFG_W6 = {(16384, 2560): (32, 256, 1, 4), (96, 2560): (16, 256, 2, 4), (13312, 2560): (16, 256, 1, 4),
          (640, 2560): (16, 256, 1, 2), (1280, 2560): (16, 256, 1, 2), (2560, 6144): (32, 256, 1, 4),
          (2560, 640): (32, 128, 1, 2)}
CFG_NV4 = {}
CFG_BG = {(336, 10240): (16, 512, 4, 4), (10240, 320): (32, 64, 1, 4), (512, 2560): (16, 256, 1, 4)}
CFG_HC_NV4 = {(336, 10240): (16, 128, 2, 20), (10240, 320): (32, 64, 4, 1)}
CFG_W8 = {(336, 10240): (32, 256, 8, 4), (10240, 320): (32, 64, 1, 8), (512, 2560): (16, 512, 1, 4)}
# The fused mixer's down projection and the unfused one (CFG_W8[(336, 10240)])
# use the same KSPLIT, so both give the same bits.
HC_DOWN_CFG = (32, 256, 8, 4)
HC_UP_CFG = (8, 64, 4)
MAX_ROWS = 16            # decode shapes: at most this many activation rows


def _say(msg):
    print(f"[fp4x] {msg}", file=sys.stderr, flush=True)


def _env(name, default=""):
    return os.environ.get(name, default)


def _on(name):
    return os.environ.get(name) == "1"


def _k_tile(k, tiles=(512, 256, 128, 64)):
    """The largest K tile of `tiles` that divides k (the last one otherwise)."""
    return next((t for t in tiles if k % t == 0), tiles[-1])


def _mx8_cfg(n, k):
    """The MXFP8 linear's cfg for an (N, K) weight: the table's, else one
    K slice with the largest K tile dividing K."""
    return CFG_MX8.get((n, k)) or (32, _k_tile(k), 1, 4)


class _Stats:
    """Call counts of the hooks, logged every `every` counted calls (the
    reference logs its dense-linear counts every 20,000 calls,
    x/fp4patch.py:22, :122-123, :135-136)."""

    def __init__(self, every=20000):
        self.every, self.n, self.total = every, {}, 0

    def count(self, key):
        self.n[key] = self.n.get(key, 0) + 1
        self.total += 1
        if self.total % self.every == 0:
            _say(f"stats {dict(sorted(self.n.items()))}")


STATS = _Stats()


class _Milestones:
    """Counts events per key and says when a count reaches one of `marks`."""

    def __init__(self, marks):
        self.marks, self.n = set(marks), {}

    def hit(self, key):
        self.n[key] = self.n.get(key, 0) + 1
        return self.n[key] in self.marks


def _capturing(torch):
    return torch.cuda.is_current_stream_capturing()


# ----------------------------------------------------------------- dense linears
class _DenseDecode:
    """State of the b12x MXFP8 linear hook (x/fp4patch.py:41-140)."""

    def __init__(self, torch, F, original):
        self.torch, self.F, self.original = torch, F, original
        self.max_rows = int(_env("FP4X_MX8_MAXM", "16"))
        self.mode = _env("FP4X_DENSE", "mx8")                         # mx8 | w6 | nv4
        self.nv4_shapes = {tuple(int(d) for d in item.split("x")) for item in _env("FP4X_NV4_SHAPES").split(",")
                           if item}
        self.qmax = int(_env("FP4X_DENSE_QMAX", "31"))
        self.clip = int(_env("FP4X_DENSE_CLIP", "0"))
        self.zero = _on("FP4X_MX8_ZERO")
        self.copies = {}                                              # id(layer) -> low-bit planes
        self.shapes_seen = set()
        for flag in ("FP4X_DENSE_STATS", "FP4X_DENSE_AWQ"):
            if _env(flag):
                _say(f"{flag} (an activation-aware quality probe of the reference) is not built here; ignored")

    def low_bit_format(self, n, k):
        return "nv4" if (n, k) in self.nv4_shapes else self.mode

    def low_bit_copy(self, layer, w, s):
        """The layer's W6 or NVFP4 copy, made on its first eager call; None
        while a graph is being captured before that."""
        planes = self.copies.get(id(layer))
        if planes is None and not _capturing(self.torch):
            F = self.F
            if self.low_bit_format(*w.shape) != "w6":
                planes = F.requantize_mx8(w, s, "nv4")              # read from the packed rows directly
            else:                                                    # with the clip search when one is set
                planes = F.requantize_mx8(w, s, "w6", qmax=self.qmax, clip_search=self.clip)
            self.copies[id(layer)] = planes
            if len(self.copies) in (1, 200):
                _say(f"dense {self.mode}: {len(self.copies)} layers have their low-bit copy")
        return planes

    def packed_rows(self, layer, source, bias):
        """(fp8 weight [N, K], e8m0 scales [N, K/32]) when this call is one the
        hook serves, else None."""
        torch = self.torch
        if layer.recipe != "mxfp8" or source.dim() != 2 or source.shape[0] > self.max_rows or bias is not None:
            return None
        pk = layer.packed
        w = pk.weight.values
        if w.dtype == torch.uint8:
            w = w.view(torch.float8_e4m3fn)
        if pk.padded_in_features != pk.in_features or w.dtype != torch.float8_e4m3fn or w.dim() != 2:
            return None
        return w, pk.weight.scale_rows.view(torch.uint8).view(w.shape[0], -1)

    def run(self, layer, source, bias):
        rows = self.packed_rows(layer, source, bias)
        if rows is None:
            STATS.count("mx8_skip")
            return self.original(layer, source, bias)
        STATS.count("mx8")
        w, s = rows
        n, k = w.shape
        F = self.F
        if self.mode != "mx8" and n < 100000:
            planes = self.low_bit_copy(layer, w, s)
            if planes is not None:
                fmt = self.low_bit_format(n, k)
                self._note(source, n, k, fmt)
                if fmt == "w6":
                    return F.w6_linear(source, *planes, CFG_W6.get((n, k)) or (32, 256, 1, 4))
                return F.nv4_linear(source, *planes, CFG_NV4.get((n, k)) or (32, _k_tile(k, (256, 128, 64)), 4))
        if self.zero:
            return self.torch.zeros((source.shape[0], n), dtype=source.dtype, device=source.device)
        self._note(source, n, k, "mx8")
        return F.mx8_linear(source, w, s, _mx8_cfg(n, k))

    def _note(self, source, n, k, fmt):
        key = (source.shape[0], n, k, fmt)
        if key not in self.shapes_seen and len(self.shapes_seen) < 64:
            self.shapes_seen.add(key)
            _say(f"dense: {source.shape[0]} x {n}x{k} served as {fmt}")


def _patch_mx8():
    import torch
    from vllm.model_executor.kernels.linear import b12x_blockscaled as BB
    import fp4x_kernels as F
    hook = _DenseDecode(torch, F, BB.B12xBlockscaledLinear.run)

    def run(self, source, bias):
        return hook.run(self, source, bias)

    BB.B12xBlockscaledLinear.run = run
    _say(f"b12x MXFP8 linears of up to {hook.max_rows} rows now run the fp4x GEMVs ({hook.mode})")


# ----------------------------------------------------------------- mixers, gates, MTP linears
class _Projection:
    """The custom op vllm::fp4x_bf16_linear(x, w, allow_w8) that the mixer,
    router-gate and MTP hooks call (x/fp4patch.py:158-195): for at most 16
    rows a quantized copy of w (made on first eager use) or w itself runs an
    fp4x GEMV; larger batches take torch's linear."""

    def __init__(self, torch, F):
        self.torch, self.F = torch, F
        self.zero = _on("FP4X_HC_ZERO")
        self.w8 = _on("FP4X_HC_W8")
        self.nv4 = _on("FP4X_HC_NV4")
        self.w6 = _on("FP4X_HC_W6")
        self.copies = {"nv4": {}, "w6": {}, "w8": {}}                # (data_ptr, shape) -> planes
        self.calls = _Milestones((1, 100, 10000))

    def copy(self, fmt, w, make):
        store = self.copies[fmt]
        key = (w.data_ptr(), tuple(w.shape))
        planes = store.get(key)
        if planes is None and not _capturing(self.torch):
            planes = store[key] = make(w)
            if fmt == "w8" and len(store) in (1, 100):
                _say(f"mixer projections: {len(store)} int8 copies made")
        return planes

    def __call__(self, x, w, allow_w8):
        F, torch = self.F, self.torch
        if self.calls.hit("op"):
            _say(f"projection op: call {self.calls.n['op']}, x {tuple(x.shape)}, w {tuple(w.shape)}")
        if x.shape[0] > MAX_ROWS:
            return torch.nn.functional.linear(x, w)
        n, k = w.shape
        if self.zero:
            return torch.zeros((x.shape[0], n), dtype=x.dtype, device=x.device)
        if allow_w8 and self.nv4:
            planes = self.copy("nv4", w, F.quantize_nv4)
            if planes is not None:
                return F.nv4_linear(x.contiguous(), *planes, CFG_HC_NV4.get((n, k)) or (32, 64, 4, 1))
        if allow_w8 and self.w6 and (n, k) != (512, 2560):
            planes = self.copy("w6", w, F.quantize_w6)
            if planes is not None:
                return F.w6_linear(x.contiguous(), *planes, (32, _k_tile(k, (256, 64)), 1, 4))
        if allow_w8 and self.w8:
            planes = self.copy("w8", w, F.quantize_w8)
            if planes is not None:
                return F.w8_linear(x.contiguous(), *planes, CFG_W8.get((n, k)) or (32, _k_tile(k, (256, 64)), 1, 4))
        return F.bf16_linear(x.contiguous(), w, CFG_BG.get((n, k)) or (32, _k_tile(k, (256, 64)), 1, 4))


class _Mixer:
    """State of the GatedResidual._mix_normalized hook (x/fp4patch.py:197-249).

    The fused mixer runs as one launch (HCFused.mix), whose up workgroups wait
    for the bottleneck with a bounded wait; a wait that gives up leaves NaN in
    that call's block_input and sets a status bit.  check_waits() reads that bit
    without blocking, from eager calls (every CHECK_EVERY-th eager mixer call,
    and every eager call of the fast head); after a give-up the hook logs and
    counts it and runs each mixer as two launches (down, then up), which wait
    for nothing.  Graphs captured before keep the launches they recorded."""

    CHECK_EVERY = 64

    def __init__(self, torch, F, HC, op, fused):
        self.torch, self.F, self.HC, self.op, self.fused = torch, F, HC, op, fused
        self.w8_mtp = _on("FP4X_HC_W8_MTP")
        self.scratch = None                                           # one HCFused for every mixer
        self.down = {}                                                # (data_ptr, shape) -> (q, s)
        self.up = {}                                                  # (data_ptr, shape) -> interleaved (q, s)
        self.single = True                                            # one launch per fused mixer
        self.timeouts = 0
        self.eager_calls = 0

    def check_waits(self):
        """Poll the single-launch mixer's status word (non-blocking, eager only);
        on a give-up, log, count and switch to two launches per mixer."""
        if self.scratch is None or not self.single or _capturing(self.torch):
            return
        if self.scratch.poll_timeouts():
            self.timeouts += 1
            self.single = False
            STATS.count("mix_timeout")
            _say(f"fused mixers: a single-launch mixer gave up waiting for its bottleneck ({self.timeouts} so far; "
                 "its block_input held NaN); each mixer now runs as two launches (graphs captured before keep "
                 "the single launch)")

    def _prepared(self, res, normalized):
        """The layer's (down, up) W8 copies and the shared scratch, prepared on
        its first eager call; None while capturing before that."""
        wd = (res.input_mix_weight_down_block_inject if res.use_combine else res.input_mix_weight_down).weight
        wu = res.input_mix_weight_up.weight
        kd, ku = (wd.data_ptr(), tuple(wd.shape)), (wu.data_ptr(), tuple(wu.shape))
        if kd in self.down and ku in self.up and self.scratch is not None:
            return self.down[kd], self.up[ku]
        if _capturing(self.torch):
            return None
        F = self.F
        if self.scratch is None:
            self.scratch = F.HCFused(normalized.device, n_down=max(336, wd.shape[0]))
        if kd not in self.down:
            self.down[kd] = F.quantize_w8(wd)
        if ku not in self.up:
            self.up[ku] = F.HCFused.interleave_up(*F.quantize_w8(wu), res.hc_count, 8)
            if len(self.up) in (1, 97):
                _say(f"fused mixers: {len(self.up)} layers prepared")
        return self.down[kd], self.up[ku]

    def fused_mix(self, res, normalized):
        planes = self._prepared(res, normalized)
        if planes is None:
            return None
        (qd, sd), (qi, si) = planes
        x = normalized.contiguous()
        # down then up, as HCFused.down + HCFused.up (x/fp4patch.py:217-218), one launch where the shapes allow
        if self.single:
            STATS.count("mix_single")
            di, _, block_input = self.scratch.mix(x, qd, sd, res.lora_rank, res.hc_count, qi, si, x, HC_DOWN_CFG,
                                                  HC_UP_CFG)
        else:
            STATS.count("mix_two")
            di, bot = self.scratch.down(x, qd, sd, res.lora_rank, res.hc_count, HC_DOWN_CFG)
            block_input = self.F.HCFused.up(bot, qi, si, x, res.hc_count, HC_UP_CFG)
        injection = di[:, res.lora_rank: res.lora_rank + res.hc_count] if res.use_combine else None
        return block_input, injection

    def mix(self, res, normalized, original):
        if res.tp_size > 1:
            STATS.count("mix_skip")
            return original(res, normalized)
        if self.scratch is not None and not _capturing(self.torch):
            self.eager_calls += 1
            if self.eager_calls % self.CHECK_EVERY == 0:
                self.check_waits()
        quantized = "mtp" not in (res._preparation_prefix or "") or self.w8_mtp
        decode = normalized.shape[0] <= MAX_ROWS
        if self.fused and quantized and decode:
            out = self.fused_mix(res, normalized)
            if out is not None:
                return out
        lr, hc = res.lora_rank, res.hc_count
        if res.use_combine:
            both = self.op(normalized, res.input_mix_weight_down_block_inject.weight, quantized)
            down, injection = both[:, :lr], both[:, lr: lr + hc]
        else:
            down, injection = self.op(normalized, res.input_mix_weight_down.weight, quantized), None
        on_gpu = decode and down.is_cuda
        # the scaled-SiLU and gate-mean epilogues: fp4x kernels (the fused mixer's
        # rounding points) for decode rows, the model's own ops otherwise
        bottleneck = self.F.hc_scaled_silu(down, lr, hc) if on_gpu else self.HC.hc_silu(down, hc)
        gate_logits = self.op(bottleneck, res.input_mix_weight_up.weight, quantized)
        block_input = (self.F.hc_gate_mean(normalized, gate_logits, hc) if on_gpu
                       else self.HC.hc_gate_mix(normalized, gate_logits, hc))
        STATS.count("mix_unfused")
        return block_input, injection


MIXERS = []              # the installed mixer hooks, whose status the fast head's eager calls also check


def _patch_linears(torch, op, mtp_w8, gate_mode):
    """UnquantizedLinearMethod.apply for the router gates (`*.mlp.gate`, at
    most 16 rows; FP4X_GATE=w8|bf16) and the MTP layers' linears (`mtp.*`,
    FP4X_MTP_W8=1) (x/fp4patch.py:251-275)."""
    from vllm.model_executor.layers.linear import UnquantizedLinearMethod
    import fp4x_kernels as F
    original = UnquantizedLinearMethod.apply
    gates = _Milestones((1, 1000))

    def apply(self, layer, x, bias=None):
        if bias is not None or layer.weight.dim() != 2:
            return original(self, layer, x, bias)
        prefix = str(getattr(layer, "prefix", ""))
        n = layer.weight.shape[0]
        rows = x.reshape(-1, x.shape[-1])
        if mtp_w8 and prefix.startswith("mtp."):
            return op(rows, layer.weight, True).view(*x.shape[:-1], n)
        if gate_mode and prefix.endswith(".mlp.gate") and rows.shape[0] <= MAX_ROWS:
            rows = rows.contiguous()
            if gates.hit("gate"):
                _say(f"router gates ({gate_mode}): call {gates.n['gate']} at {prefix}, {rows.shape[0]} rows")
            if gate_mode == "w8":
                y = op(rows, layer.weight, True)
            else:
                y = F.bf16_linear(rows, layer.weight, CFG_BG.get(tuple(layer.weight.shape)) or (16, 256, 1, 4))
            return y.view(*x.shape[:-1], n)
        return original(self, layer, x, bias)

    UnquantizedLinearMethod.apply = apply
    _say(f"unquantized linears hooked: MTP int8 {'on' if mtp_w8 else 'off'}, router gates {gate_mode or 'off'}")


def _patch_hc():
    import torch
    from vllm.models.qwen4_exp.nvidia import hyperconnection as HC
    from vllm.utils.torch_utils import direct_register_custom_op
    import fp4x_kernels as F

    projection = _Projection(torch, F)

    def fp4x_bf16_linear(x: torch.Tensor, w: torch.Tensor, allow_w8: bool) -> torch.Tensor:
        return projection(x, w, allow_w8)

    def fp4x_bf16_linear_fake(x: torch.Tensor, w: torch.Tensor, allow_w8: bool) -> torch.Tensor:
        return x.new_empty((x.shape[0], w.shape[0]))

    direct_register_custom_op(op_name="fp4x_bf16_linear", op_func=fp4x_bf16_linear,
                              fake_impl=fp4x_bf16_linear_fake)
    op = torch.ops.vllm.fp4x_bf16_linear
    original = HC.GatedResidual._mix_normalized
    mixer = _Mixer(torch, F, HC, op, fused=projection.w8 and _on("FP4X_HC_FUSED"))
    MIXERS.append(mixer)

    def _mix_normalized(self, normalized):
        return mixer.mix(self, normalized, original)

    HC.GatedResidual._mix_normalized = _mix_normalized
    _say(f"hyper-connection mixers of up to {MAX_ROWS} rows now run the fp4x GEMVs"
         f"{' (fused, int8)' if mixer.fused else ''}")
    mtp_w8, gate_mode = _on("FP4X_MTP_W8"), _env("FP4X_GATE")
    if mtp_w8 or gate_mode:
        _patch_linears(torch, op, mtp_w8, gate_mode)


# ----------------------------------------------------------------- target LM head
class _FastHead:
    """State of the target head hook (x/fp4patch.py:337-393)."""

    def __init__(self, torch, F, original):
        self.torch, self.F, self.original = torch, F, original
        self.C = int(_env("FP4X_HEAD_C", "512"))
        self.G = int(_env("FP4X_HEAD_G", "16"))
        self.int2 = _env("FP4X_HEAD_COARSE", "int2") == "int2"
        self.disabled = False
        self.ready = False

    def build(self, model, h):
        """First eager call: the coarse copy, then the reference's self-check
        against the original head (argmax agreement 1.0, top-20 max |d| <=
        1e-2), which disables the fast head when it fails."""
        torch, F = self.torch, self.F
        lp = model.logits_processor
        if lp.scale != 1.0 or lp.soft_cap is not None:
            self.disabled = True
            _say("fast head: the logits processor scales or soft-caps, keeping the original head")
            return
        pk = model.lm_head.b12x_mxfp8_packed_weight
        self.w = pk.weight.values
        self.s = pk.weight.scale_rows.view(torch.uint8).view(self.w.shape[0], -1)
        # the coarse copy, read from the packed MXFP8 rows (no fp32 copy of the head)
        self.coarse = (F.requantize_mx8(self.w, self.s, "int2", group=self.G) if self.int2
                       else F.requantize_mx8(self.w, self.s, "nv4"))
        self.ready = True
        want = self.original(model, h)
        got = self.logits(h)
        argmax_agree = (got.argmax(-1) == want.argmax(-1)).float().mean().item()
        top = torch.topk(want.float(), 20, dim=-1).indices
        top_err = (got.float().gather(1, top) - want.float().gather(1, top)).abs().max().item()
        _say(f"fast head ready (C={self.C}, G={self.G}): argmax agreement {argmax_agree:.3f}, "
             f"top-20 max |d| {top_err:.2e} against the original head")
        if argmax_agree < 1.0 or top_err > 1e-2:
            self.disabled = True
            _say("fast head: self-check not passed, keeping the original head")

    def logits(self, h):
        F = self.F
        if self.int2:
            P, S = self.coarse
            # int2_logits + top-C in one call (the coarse kernel also yields the top-k's slice maxima)
            coarse, idx = F.int2_topk(h, P, S, self.w.shape[0], self.C, sorted=False)
        else:
            P, S, gs = self.coarse
            coarse = F.nv4_linear(h, P, S, gs, (32, 256, 4))
            idx = F.topk_rows(coarse, self.C)
        return F.refine_mx8_(coarse, h, idx, self.w, self.s)          # exact rows scattered in place

    def compute(self, model, hidden_states):
        h = hidden_states
        for mixer in MIXERS:                          # once per step: the head runs eagerly
            mixer.check_waits()
        if self.disabled or h.dim() != 2 or not 0 < h.shape[0] <= MAX_ROWS:
            STATS.count("head_skip")
            return self.original(model, hidden_states)
        if not self.ready:
            if _capturing(self.torch):
                return self.original(model, hidden_states)
            self.build(model, h.contiguous())
            if self.disabled:
                return self.original(model, hidden_states)
        STATS.count("head")
        return self.logits(h.contiguous())


def _patch_fast_head():
    import torch
    from vllm.models.qwen4_exp.nvidia import model as MD
    import fp4x_kernels as F
    head = _FastHead(torch, F, MD.Qwen4ExpForCausalLM.compute_logits)

    def compute_logits(self, hidden_states):
        return head.compute(self, hidden_states)

    MD.Qwen4ExpForCausalLM.compute_logits = compute_logits
    _say(f"target LM head of up to {MAX_ROWS} rows: INT2 coarse + top-{head.C} exact MXFP8 rescore")


# ----------------------------------------------------------------- draft head
# 1 / FP4X_DRAFT_TSCALE as a one-element device tensor per device: the scatter
# reads it on the device, so captured graphs pick up a changed value.
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
    INT2 coarse over the subset in fp32, its top dc (one int2_topk call), their
    exact NVFP4 logits; else the NVFP4 GEMV over the whole subset.
    [x/fp4patch.py:309-330]"""
    import torch
    if dc and h.shape[0] <= MAX_ROWS:
        # the top dc of the fp32 coarse logits (int2_logits' default dtype, as x/fp4patch.py:313-314 selects)
        _, cand = F.int2_topk(h, *st["c"], st["idx"].numel(), dc, out_dtype=torch.float32, sorted=False)
        # their exact NVFP4 logits scattered into the -inf row: one launch (refine_nv4 + scatter_draft)
        return F.draft_nv4(h, cand, st["w"], st["s"], st["gs"], st["idx"], vocab, inv_t)
    sub = F.nv4_linear(h, st["w"], st["s"], st["gs"], cfg)
    full = torch.full((h.shape[0], vocab), float("-inf"), dtype=sub.dtype, device=sub.device)
    full.index_copy_(1, st["idx"], sub)
    return full


def _unswizzle_nv4_scales(torch, sc):
    """b12x's NVFP4 scale tiles (128 rows x 4 scale columns, stored 32 x 4 x 4)
    back to row-major [n, kb] e4m3 (x/fp4patch.py:296)."""
    n, kb = sc.shape
    rows = sc.view(torch.uint8).reshape(n // 128, kb // 4, 32, 4, 4).transpose(1, 3).reshape(n, kb)
    return rows.view(torch.float8_e4m3fn)


def _patch_draft_vocab():
    import torch
    from vllm.models.qwen4_exp.nvidia import mtp as MTP
    import fp4x_kernels as F
    path = os.environ["FP4X_DRAFT_VOCAB"]
    cfg = tuple(int(v) for v in _env("FP4X_DRAFT_CFG", "32,256,4").split(","))
    dc = int(_env("FP4X_DRAFT_INT2", "0"))
    tscale = float(_env("FP4X_DRAFT_TSCALE", "1.0"))
    G = int(_env("FP4X_DRAFT_INT2_G", "16"))
    original = MTP.Qwen4ExpMTP.compute_logits

    def build(self, device):
        lm = self.lm_head
        vocab = lm.weight.shape[0]
        listed = {int(tok) for tok in open(path) if tok.strip()}
        tail = set(range(lm.org_vocab_size - 320, lm.org_vocab_size))   # the last 320 ids are always served
        ids = torch.tensor([i for i in sorted(listed | tail) if i < vocab], device=device, dtype=torch.long)
        self._fx = _draft_prepare(F, lm.weight.data, _unswizzle_nv4_scales(torch, lm.weight_scale.data),
                                  lm.weight_global_scale.item(), ids, dc, G)
        self._fx_vocab = vocab
        _say(f"draft head over {ids.numel()} of {vocab} ids"
             + (f": INT2 coarse, exact NVFP4 rescore of the top {dc}" if dc else ": NVFP4 GEMV over the subset"))

    def compute_logits(self, hidden_states, spec_step_idx=0):
        if getattr(self, "_fx", None) is None:
            if _capturing(torch) or getattr(self.lm_head, "weight", None) is None:
                return original(self, hidden_states, spec_step_idx)
            build(self, hidden_states.device)
        h = hidden_states.reshape(-1, hidden_states.shape[-1]).contiguous()
        inv_t = None
        if tscale != 1.0:
            inv_t = _DRAFT_INV_T.get(h.device)
            if inv_t is None:
                inv_t = _DRAFT_INV_T[h.device] = torch.full((1,), 1.0 / tscale, dtype=torch.float32, device=h.device)
        return _draft_logits(F, h, self._fx, self._fx_vocab, dc, cfg, inv_t)

    MTP.Qwen4ExpMTP.compute_logits = compute_logits
    _say(f"MTP draft head restricted to the ids of {path}")


# ----------------------------------------------------------------- entry point
# Switches of reference patches this plugin does not implement (disk PLE
# embeddings, the drafter weight swap, MoE ablations, graph debugging):
# reported, not acted on.
_NOT_BUILT = ("FP4X_KEEP_GRAPH", "FP4X_MOE_ZERO", "FP4X_MOE_TAU", "FP4X_MTP_PATCH", "FP4X_PLE_SPIN",
              "FP4X_PLE_EARLY", "FP4X_PLE_QD")

# (switch, test of its value, installer), in the reference's order of installation
_PATCHES = (
    ("FP4X_FAST_HEAD", _on, _patch_fast_head),
    ("FP4X_DRAFT_VOCAB", lambda name: bool(_env(name)), _patch_draft_vocab),
    ("FP4X_MX8", _on, _patch_mx8),
    ("FP4X_HC", _on, _patch_hc),
)


def register():
    """vLLM general-plugin entry point: install the hooks the FP4X_* switches
    ask for.  An installer that fails is reported and skipped, so a missing
    optional piece never stops the server."""
    for flag in _NOT_BUILT:
        if _env(flag):
            _say(f"{flag}: that reference patch is not implemented by this plugin; ignored")
    for flag, wanted, install in _PATCHES:
        if not wanted(flag):
            continue
        try:
            install()
        except Exception as e:
            _say(f"{flag}: could not install ({type(e).__name__}: {e}); skipped")
