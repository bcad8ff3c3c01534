"""Decode GEMVs for MI355X (gfx950): the fp4patch plugin's kernel module.

Same public names, call signatures, packed layouts and return values as the
plugin's Triton module (x/fp4x_kernels.py); every GEMV runs a hand-written HIP
kernel from libfp4x.so through its C ABI (include/fp4x.h), launched on the
current torch stream.  There is no fallback: without the built library on a
GPU these functions raise.

`cfg` tuples keep the reference's meaning for the parts that change results
or preconditions: KSPLIT is the number of K slices whose fp32 partials are
summed (in slice order, deterministically), and the reference's shape
assertion on (K, KSPLIT, BK) is kept.  Tile sizes and warp counts are GB10
Triton knobs; the HIP kernels choose their own gfx950 layout.

Weight preparation: quantize_* and requantize_* run as HIP kernels on device
tensors (libfp4x.so's quantizers, bit-exact with the reference's fp32 torch
expressions) and as those torch expressions on CPU tensors; mx8_dequant is a
HIP kernel; dequant_int2, dequant_nv4 and interleave_up are torch
expressions.  Each runs once per weight at load time.
"""
import torch

import _fp4x as _L

__all__ = [
    "mx8_linear", "bf16_linear", "nv4_linear", "w8_linear", "w6_linear", "int2_logits", "refine_mx8_", "refine_nv4",
    "scatter_draft", "draft_nv4",
    "topk_rows", "int2_topk", "w8_linear_layers", "HCFused", "hc_scaled_silu", "hc_gate_mean",
    "quantize_w8", "quantize_w6", "quantize_nv4", "quantize_int2", "quantize_mx8",
    "mx8_dequant", "dequant_int2", "dequant_nv4", "dequant_operand", "requantize_mx8", "requantize_nv4", "ORDER",
]

MAX_M = 16  # rows per launch; larger M runs as consecutive 16-row launches


# ----------------------------------------------------------------- plumbing
class _Scratch:
    """Per-device split-K scratch: fp32 slice slots (fully rewritten by every
    call) and int32 tickets (zero between calls; each call re-arms them)."""

    def __init__(self, device):
        self.device = device
        self.part = torch.empty(1 << 22, dtype=torch.float32, device=device)
        self.tickets = torch.zeros(1 << 16, dtype=torch.int32, device=device)
        self._old = []

    def get(self, floats, tickets):
        if floats > self.part.numel() or tickets > self.tickets.numel():
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("fp4x: split-K scratch too small during graph capture; run once eagerly first")
            self._old.append((self.part, self.tickets))
            if floats > self.part.numel():
                self.part = torch.empty(floats, dtype=torch.float32, device=self.device)
            if tickets > self.tickets.numel():
                self.tickets = torch.zeros(tickets, dtype=torch.int32, device=self.device)
        return self.part, self.tickets


_SCRATCH = {}


def _scratch(device, fmt, M, N, K, ks, batch=1):
    if ks == 1:
        return None, None
    floats, tickets = _L.splitk_sizes(fmt, M, N, K, ks, batch)
    key = (device.type, device.index)
    sc = _SCRATCH.get(key)
    if sc is None:
        sc = _SCRATCH[key] = _Scratch(device)
    return sc.get(floats, tickets)


def _need_cuda(*ts):
    for t in ts:
        if t is not None and torch.is_tensor(t) and not t.is_cuda:
            raise RuntimeError("fp4x: HIP kernels need GPU tensors")


def _act(x2):
    """bf16 activations with unit column stride, 16-byte aligned rows."""
    if x2.dtype != torch.bfloat16:
        raise TypeError(f"fp4x: activations must be bfloat16, got {x2.dtype}")
    if x2.dim() != 2:
        raise ValueError("fp4x: activations must be 2-D [M, K]")
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16 or x2.stride(0) < x2.shape[1]:
        x2 = x2.contiguous()
        if x2.data_ptr() % 16:
            x2 = x2.clone()
    return x2


def _rows_blocks(M):
    return range(0, M, MAX_M)


def _ptr(t):
    return _L.ptr(t)


def _dt(dtype):
    code = _L.DTYPE_CODE.get(dtype)
    if code is None:
        raise TypeError(f"fp4x: unsupported output dtype {dtype}")
    return code


def _check_split(k, cfg, ks_idx=2, bk_idx=1):
    KS = cfg[ks_idx] if len(cfg) > ks_idx else 1
    BK = cfg[bk_idx]
    assert k % KS == 0 and (k // KS) % BK == 0, (k, cfg)
    return KS


def _linear(fn, fmt, x2, n, k, ks, out_dtype, args):
    """Run a dense GEMV entry point over 16-row blocks of x2."""
    x2 = _act(x2)
    m = x2.shape[0]
    if x2.shape[1] != k:
        raise ValueError(f"fp4x: activation K={x2.shape[1]} does not match weight K={k}")
    out = torch.empty((m, n), dtype=out_dtype, device=x2.device)
    st = _L.stream_of(x2)
    for m0 in _rows_blocks(m):
        mb = min(MAX_M, m - m0)
        xb, ob = x2[m0:m0 + mb], out[m0:m0 + mb]
        part, tick = _scratch(x2.device, fmt, mb, n, k, ks)
        _L.check(fn(_ptr(xb), xb.stride(0), *args, _ptr(ob), _dt(out_dtype), mb, n, k, ks, _ptr(part), _ptr(tick), st),
                 fn.__name__)
    return out


# ----------------------------------------------------------------- GEMVs
def mx8_linear(x2, w8, s, cfg, out_dtype=torch.bfloat16):
    """y = x2 . bf16(e4m3(w8) * 2^(s-127))^T; w8 [N, K] fp8/uint8, s uint8 [N, K/32]."""
    _need_cuda(x2, w8, s)
    n, k = w8.shape
    ks = _check_split(k, cfg)
    return _linear(_L.lib().fp4x_mx8_linear, _L.FMT_MX8, x2, n, k, ks, out_dtype, (_ptr(w8), _ptr(s)))


def bf16_linear(x2, w, cfg, out_dtype=torch.bfloat16):
    """y = x2 . w^T with bf16 weights w [N, K]."""
    _need_cuda(x2, w)
    if w.dtype != torch.bfloat16 or w.stride(1) != 1 or w.stride(0) != w.shape[1]:
        w = w.to(torch.bfloat16).contiguous()
    n, k = w.shape
    ks = _check_split(k, cfg)
    return _linear(_L.lib().fp4x_bf16_linear, _L.FMT_BF16, x2, n, k, ks, out_dtype, (_ptr(w),))


def w8_linear(x2, q, s, cfg, out_dtype=torch.bfloat16):
    """y = x2 . bf16(q * s)^T; q int8 [N, K], s fp32 (or fp16) [N, K/64]."""
    _need_cuda(x2, q, s)
    n, k = q.shape
    ks = _check_split(k, cfg)
    sdt = _L.DT_F16 if s.dtype == torch.float16 else _L.DT_F32
    if s.dtype not in (torch.float16, torch.float32):
        raise TypeError("fp4x: W8 scales must be fp32 or fp16")
    fmt = _L.FMT_W8_F16 if sdt == _L.DT_F16 else _L.FMT_W8_F32
    return _linear(_L.lib().fp4x_w8_linear, fmt, x2, n, k, ks, out_dtype, (_ptr(q), _ptr(s), sdt))


def w6_linear(x2, L, H, S, cfg, out_dtype=torch.bfloat16):
    """y = x2 . bf16((code - 32) * S)^T; L [N, K/2], H [N, K/4], S fp16 [N, K/32]."""
    _need_cuda(x2, L, H, S)
    n, k = L.shape[0], L.shape[1] * 2
    ks = _check_split(k, cfg)
    return _linear(_L.lib().fp4x_w6_linear, _L.FMT_W6, x2, n, k, ks, out_dtype, (_ptr(L), _ptr(H), _ptr(S)))


def nv4_linear(x2, wp, s, gs, cfg=(32, 256, 4), out_dtype=torch.bfloat16):
    """y = gs * (x2 . bf16(e2m1(wp) * e4m3(s))^T); cfg (BN, BK, num_warps[, KSPLIT])."""
    _need_cuda(x2, wp, s)
    n, k = wp.shape[0], wp.shape[1] * 2
    ks = _check_split(k, cfg, ks_idx=3)
    return _linear(_L.lib().fp4x_nv4_linear, _L.FMT_NV4, x2, n, k, ks, out_dtype, (_ptr(wp), _ptr(s), float(gs)))


def w8_linear_layers(x3, q3, s3, out_dtype=torch.bfloat16):
    """Independent W8 GEMVs of L layers in one launch: x3 [L, M, K] bf16,
    q3 [L, N, K] int8, s3 [L, N, K/64] fp32/fp16 -> [L, M, N] (e.g. every
    router gate of a decode step)."""
    _need_cuda(x3, q3, s3)
    if x3.dtype != torch.bfloat16:
        raise TypeError("fp4x: activations must be bfloat16")
    x3, q3, s3 = x3.contiguous(), q3.contiguous(), s3.contiguous()
    Ly, m, k = x3.shape
    n = q3.shape[1]
    if m > MAX_M:
        raise ValueError("fp4x: w8_linear_layers takes at most 16 rows per layer")
    sdt = _L.DT_F16 if s3.dtype == torch.float16 else _L.DT_F32
    out = torch.empty((Ly, m, n), dtype=out_dtype, device=x3.device)
    _L.check(_L.lib().fp4x_w8_linear_layers(_ptr(x3), k, m * k, _ptr(q3), n * k, _ptr(s3), sdt, n * (k // 64),
                                            _ptr(out), _dt(out_dtype), m * n, Ly, m, n, k, 1, None, None,
                                            _L.stream_of(x3)), "w8_linear_layers")
    return out


def int2_logits(x, P, S, N, BN=64, BK=512, nw=4, RS=None, out_dtype=torch.float32):
    """INT2 coarse logits [M, N]: x . bf16((code - 1.5) * S)^T (times RS[n]).
    S fp16 [N, K/G] or e4m3 with a per-row fp32 RS."""
    _need_cuda(x, P, S)
    x = x.to(torch.bfloat16).contiguous()
    m, k = x.shape
    G = k // S.shape[1]
    sfmt = _L.DT_E4M3 if S.dtype == torch.float8_e4m3fn else _L.DT_F16
    out = torch.empty((m, N), dtype=out_dtype, device=x.device)
    st = _L.stream_of(x)
    for m0 in _rows_blocks(m):
        mb = min(MAX_M, m - m0)
        _L.check(_L.lib().fp4x_int2_logits(_ptr(x[m0:]), k, _ptr(P), _ptr(S), sfmt,
                                           _ptr(RS) if RS is not None else None, _ptr(out[m0:]), _dt(out_dtype),
                                           mb, N, k, G, st), "int2_logits")
    return out


def int2_topk(x, P, S, N, C, RS=None, out_dtype=torch.bfloat16, sorted=True):
    """The coarse stage of the fast head (bf16) or of the draft head (fp32):
    (coarse [M, N], idx int64 [M, C]) = (int2_logits(x, P, S, N, RS=RS,
    out_dtype=out_dtype), topk_rows(coarse, C)), in one call that lets the
    coarse kernel produce the top-k's slice maxima.  sorted=False: the same
    index set per row in an unspecified order, for callers that only scatter
    at these indices (where the selection can skip its sort, increasing index
    order)."""
    _need_cuda(x, P, S)
    x = x.to(torch.bfloat16).contiguous()
    m, k = x.shape
    G = k // S.shape[1]
    sfmt = _L.DT_E4M3 if S.dtype == torch.float8_e4m3fn else _L.DT_F16
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("fp4x: int2_topk gives bf16 or fp32 coarse logits")
    per16 = 16 // torch.empty((), dtype=out_dtype).element_size()
    ld = -(-N // per16) * per16
    coarse = torch.empty((m, ld), dtype=out_dtype, device=x.device)[:, :N]
    idx = torch.empty((m, C), dtype=torch.int64, device=x.device)
    st = _L.stream_of(x)
    for m0 in _rows_blocks(m):
        mb = min(MAX_M, m - m0)
        nbytes = _L.lib().fp4x_topk_workspace_size(mb, N)
        ws = _topk_workspace(x.device, nbytes)
        _L.check(_L.lib().fp4x_int2_topk(_ptr(x[m0:]), k, _ptr(P), _ptr(S), sfmt,
                                         _ptr(RS) if RS is not None else None, _ptr(coarse[m0:]), _dt(out_dtype), ld,
                                         mb, N, k, G, C, _ptr(idx[m0:]), 0 if sorted else 1, _ptr(ws), nbytes, st),
                 "int2_topk")
    return coarse, idx


def topk_rows(logits, C):
    """Indices [M, C] (int64) of the C largest logits (bf16 or fp32) of each
    row, in the order (value desc, index asc) — the selection the fast head
    and the draft head take with torch.topk, with a defined tie order."""
    _need_cuda(logits)
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("fp4x: topk_rows takes bf16 or fp32 logits")
    m, v = logits.shape
    per16 = 16 // logits.element_size()
    vr = -(-v // per16) * per16                    # rows are read in 16-byte items
    end = (logits.storage_offset() + (m - 1) * logits.stride(0) + vr) * logits.element_size()
    if (logits.stride(1) != 1 or logits.stride(0) % per16 or logits.data_ptr() % 16
            or (m and end > logits.untyped_storage().nbytes())):
        padded = torch.empty((m, vr), dtype=logits.dtype, device=logits.device)
        padded[:, :v] = logits
        logits = padded
    idx = torch.empty((m, C), dtype=torch.int64, device=logits.device)
    nbytes = _L.lib().fp4x_topk_workspace_size(m, v)
    ws = _topk_workspace(logits.device, nbytes)
    _L.check(_L.lib().fp4x_topk_rows(_ptr(logits), _dt(logits.dtype), logits.stride(0), m, v, C, _ptr(idx), _ptr(ws),
                                     nbytes, _L.stream_of(logits)), "topk_rows")
    return idx


_TOPK_WS = {}
_TOPK_WS_OLD = []


def _topk_workspace(device, nbytes):
    """Top-k workspace per device, grown on demand and reused (calls on one
    device must be stream-ordered).  A replaced buffer is kept alive, since
    a graph captured earlier may still address it; growing it during a
    capture raises (the capture would address memory sized for this call
    only), so run the largest shape eagerly once before capturing."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    ws = _TOPK_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("fp4x: top-k workspace too small during graph capture; run the largest shape "
                               "once eagerly first")
        if ws is not None:
            _TOPK_WS_OLD.append(ws)
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)
        _TOPK_WS[key] = ws
    return ws


def refine_mx8_(out, x, idx, w8, s_u8, BC=16, BK=256, nw=4):
    """Rescore the candidates in place and return out: for each row m and
    candidate c, out[m, idx[m, c]] becomes the dot product of x[m] with the
    dequantized MXFP8 weight row idx[m, c] (products exact in fp32, summed
    with fp32 fma in the rescore kernel's fixed order), cast to out's dtype."""
    _need_cuda(out, x, idx, w8, s_u8)
    x = x.to(torch.bfloat16).contiguous()
    idx = idx.to(torch.int64).contiguous()
    m, C = idx.shape
    K = x.shape[1]
    if out.stride(1) != 1:
        raise ValueError("fp4x: refine_mx8_ needs out with unit column stride")
    _L.check(_L.lib().fp4x_refine_mx8(_ptr(out), _dt(out.dtype), out.stride(0), _ptr(x), _ptr(idx), m, C, _ptr(w8),
                                      _ptr(s_u8), K, out.shape[1], _L.stream_of(x)), "refine_mx8")
    return out


def refine_nv4(x, idx, wp, s, gs, BC=16, BK=256, nw=4):
    """fp32 [M, C]: for each row m and candidate c, gs times the dot product of
    x[m] with the dequantized NVFP4 weight row idx[m, c] (exact products,
    fp32 fma in the rescore kernel's fixed order); NaN for a candidate
    outside [0, V)."""
    _need_cuda(x, idx, wp, s)
    x = x.to(torch.bfloat16).contiguous()
    idx = idx.to(torch.int64).contiguous()
    m, C = idx.shape
    K = x.shape[1]
    out = torch.empty((m, C), dtype=torch.float32, device=x.device)
    _L.check(_L.lib().fp4x_refine_nv4(_ptr(out), _ptr(x), _ptr(idx), m, C, _ptr(wp), _ptr(s), float(gs), K,
                                      wp.shape[0], _L.stream_of(x)), "refine_nv4")
    return out


def scatter_draft(vals, cand, ids, vocab, inv_t=None):
    """Draft logits [M, vocab] bf16: -inf except column ids[cand[m, c]] of row m,
    which holds bf16(vals[m, c] * inv_t) (inv_t: a one-element fp32 device
    tensor, or None for no scaling).  One launch for the reference's
    torch.full + ids[cand] + (vals * inv_t).to(bf16) + scatter_
    (x/fp4patch.py:316-320)."""
    _need_cuda(vals, cand, ids)
    vals = vals.to(torch.float32).contiguous()
    cand = cand.to(torch.int64).contiguous()
    ids = ids.to(torch.int64).contiguous()
    if inv_t is not None:
        _need_cuda(inv_t)
        if inv_t.dtype != torch.float32 or inv_t.numel() != 1:
            raise ValueError("fp4x: scatter_draft needs inv_t as one fp32 element")
    if vals.shape != cand.shape or vals.dim() != 2:
        raise ValueError("fp4x: scatter_draft needs vals and cand of one [M, C] shape")
    m, C = cand.shape
    out = torch.empty((m, vocab), dtype=torch.bfloat16, device=vals.device)
    _L.check(_L.lib().fp4x_scatter_draft(_ptr(out), out.stride(0), _ptr(vals), _ptr(cand), _ptr(ids), ids.numel(),
                                         None if inv_t is None else _ptr(inv_t), m, C, vocab, _L.stream_of(vals)),
             "scatter_draft")
    return out


def draft_nv4(x, cand, wp, s, gs, ids, vocab, inv_t=None):
    """Draft logits [M, vocab] bf16 from the candidates in one launch:
    scatter_draft(refine_nv4(x, cand, wp, s, gs), cand, ids, vocab, inv_t),
    bit for bit (wp / s: the subset's NVFP4 rows, one per entry of ids)."""
    _need_cuda(x, cand, wp, s, ids)
    x = x.to(torch.bfloat16).contiguous()
    cand = cand.to(torch.int64).contiguous()
    ids = ids.to(torch.int64).contiguous()
    if inv_t is not None:
        _need_cuda(inv_t)
        if inv_t.dtype != torch.float32 or inv_t.numel() != 1:
            raise ValueError("fp4x: draft_nv4 needs inv_t as one fp32 element")
    if cand.dim() != 2 or cand.shape[0] != x.shape[0] or wp.shape[0] != ids.numel():
        raise ValueError("fp4x: draft_nv4 needs cand [M, C] for x [M, K] and one ids entry per weight row")
    m, C = cand.shape
    out = torch.empty((m, vocab), dtype=torch.bfloat16, device=x.device)
    _L.check(_L.lib().fp4x_draft_nv4(_ptr(out), out.stride(0), _ptr(x), _ptr(cand), _ptr(ids), ids.numel(),
                                     _ptr(wp), _ptr(s), float(gs), None if inv_t is None else _ptr(inv_t), m, C,
                                     x.shape[1], vocab, _L.stream_of(x)), "draft_nv4")
    return out


# ----------------------------------------------------------------- mixer
class HCFused:
    """Fused hyper-connection mixer (two kernels per mixer).  One scratch per
    process (split-K slots + tile tickets) serves every mixer: calls must be
    stream-ordered, and each call leaves the tickets re-armed."""

    def __init__(self, device, n_down=336, max_m=16, bn=32, max_ksplit=16):
        self.n_down, self.max_m, self.max_ksplit = n_down, max_m, max_ksplit
        self.part = torch.zeros(max_ksplit * MAX_M * n_down, dtype=torch.float32, device=device)
        # one ticket per 16-row tile (the single-launch mixer: one per 128-byte
        # line, 2 * n_down ints); its count, status word and one 128-byte flag
        # line per workgroup (at most one workgroup per CU) in the last
        # 32 * (cus + 1) ints, at the same place for every shape
        cus = torch.cuda.get_device_properties(device).multi_processor_count
        self.tickets = torch.zeros(2 * max(n_down, 16) + 64 + 32 * (cus + 1), dtype=torch.int32, device=device)
        self._status_at = (self.tickets.numel() - 32 * (cus + 1)) // 32 * 32 + 1
        self._poll_host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self._poll_event = None

    def down(self, x, q, s, lr, hc, cfg=(32, 512, 4, 4)):
        """(di bf16 [M, N], bot bf16 [M, lr]) = split-K W8 GEMV + cast + scaled SiLU."""
        _need_cuda(x, q, s)
        KS = cfg[2]
        x = _act(x)
        m, k = x.shape
        n = q.shape[0]
        if m > min(self.max_m, MAX_M) or n > self.n_down or KS > self.max_ksplit:
            raise ValueError(f"fp4x HCFused.down: M={m} N={n} KSPLIT={KS} exceed the scratch "
                             f"(max_m={self.max_m}, n_down={self.n_down}, max_ksplit={self.max_ksplit})")
        di = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
        bot = torch.empty((m, lr), dtype=torch.bfloat16, device=x.device)
        sdt = _L.DT_F16 if s.dtype == torch.float16 else _L.DT_F32
        _L.check(_L.lib().fp4x_hc_down(_ptr(x), x.stride(0), _ptr(q), _ptr(s), sdt, _ptr(di), _ptr(bot), m, n, k, lr,
                                       hc, KS, _ptr(self.part), _ptr(self.tickets), _L.stream_of(x)), "hc_down")
        return di, bot

    def mix(self, x, qd, sd, lr, hc, qi, si, normalized, cfg=(32, 256, 4, 4), up_cfg=(8, 64, 4)):
        """(di, bot, block_input) = down(...) then up(bot, ...), bit-identical to the two calls
        (x/fp4patch.py:217-218), in one launch when both halves take their planned decompositions."""
        _need_cuda(x, qd, sd, qi, si, normalized)
        KS, BJ = cfg[2], up_cfg[0]
        x = _act(x)
        m, k = x.shape
        n = qd.shape[0]
        if m > min(self.max_m, MAX_M) or n > self.n_down or KS > self.max_ksplit:
            raise ValueError(f"fp4x HCFused.mix: M={m} N={n} KSPLIT={KS} exceed the scratch "
                             f"(max_m={self.max_m}, n_down={self.n_down}, max_ksplit={self.max_ksplit})")
        if qi.shape[1] != lr or sd.dtype != si.dtype:
            raise ValueError("fp4x HCFused.mix: up weights must have K = lr and the down weights' scale dtype")
        nh = qi.shape[0]
        h = nh // hc
        if normalized.stride(1) != 1:
            normalized = normalized.contiguous()
        di = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
        bot = torch.empty((m, lr), dtype=torch.bfloat16, device=x.device)
        out = torch.empty((m, h), dtype=torch.bfloat16, device=x.device)
        sdt = _L.DT_F16 if sd.dtype == torch.float16 else _L.DT_F32
        _L.check(_L.lib().fp4x_hc_mix(_ptr(x), x.stride(0), _ptr(qd), _ptr(sd), sdt, _ptr(di), _ptr(bot), m, n, k, lr,
                                      hc, KS, _ptr(self.part), _ptr(self.tickets), self.tickets.numel(), _ptr(qi),
                                      _ptr(si), _ptr(normalized), normalized.stride(0), _ptr(out), h, BJ,
                                      _L.stream_of(x)), "hc_mix")
        self._mixed = True
        return di, bot, out

    def wait_timeouts(self, clear=True):
        """True if a single-launch mixer call since the last check gave up
        waiting for its bottleneck (bit 0 of the device status word), or found
        a down tile's partials off its closer's XCD (bit 1); that call's
        outputs hold NaN.  Reads the status word: synchronizes the stream."""
        at = self._status_at
        if not getattr(self, "_mixed", False):
            return False
        hit = bool(int(self.tickets[at].item()) & 3)
        if clear and hit:
            self.tickets[at].zero_()
        return hit

    def poll_timeouts(self):
        """wait_timeouts without blocking: True if the status word copied by an
        earlier poll showed a give-up.  Each poll whose previous copy has
        arrived queues, on the current stream after the work already there, a
        copy of the word to pinned host memory and the word's clear; so a
        give-up is reported by the first poll after its copy arrives.  Eager
        use only (the copy and the clear must not be captured)."""
        if not getattr(self, "_mixed", False):
            return False
        hit = False
        if self._poll_event is not None:
            if not self._poll_event.query():
                return False                                   # the last copy is still in flight
            hit = bool(int(self._poll_host[0]) & 3)
        at = self._status_at
        self._poll_host.copy_(self.tickets[at:at + 1], non_blocking=True)
        self.tickets[at:at + 1].zero_()
        self._poll_event = torch.cuda.Event()
        self._poll_event.record()
        return hit

    @staticmethod
    def interleave_up(q, s, hc, bj):
        """Permute the up projection's rows [hc*H, K] (and their scales): stored
        row t*(hc*bj) + s*bj + j holds original row s*H + t*bj + j, so the hc
        stream rows of output columns t*bj .. t*bj + bj - 1 are one block."""
        n = q.shape[0]
        h = n // hc
        idx = torch.arange(n, device=q.device).view(hc, h // bj, bj).permute(1, 0, 2).reshape(-1)
        return q[idx].contiguous(), s[idx].contiguous()

    @staticmethod
    def up(bot, qi, si, normalized, hc, cfg=(8, 64, 8)):
        """block_input bf16 [M, H] = gate/stream-mean epilogue of the interleaved up GEMV."""
        _need_cuda(bot, qi, si, normalized)
        BJ = cfg[0]
        bot = _act(bot)
        m, k = bot.shape
        n = qi.shape[0]
        h = n // hc
        if normalized.stride(1) != 1:
            normalized = normalized.contiguous()
        out = torch.empty((m, h), dtype=torch.bfloat16, device=bot.device)
        sdt = _L.DT_F16 if si.dtype == torch.float16 else _L.DT_F32
        _L.check(_L.lib().fp4x_hc_up(_ptr(bot), bot.stride(0), _ptr(qi), _ptr(si), sdt, _ptr(normalized),
                                     normalized.stride(0), _ptr(out), m, k, h, hc, BJ, _L.stream_of(bot)), "hc_up")
        return out


def hc_scaled_silu(d, lr, hc):
    """bot [M, lr] = bf16(sc * sigmoid(sc)), sc = bf16(d / hc) (unfused mixer epilogue)."""
    _need_cuda(d)
    if d.stride(1) != 1:
        d = d.contiguous()
    m = d.shape[0]
    bot = torch.empty((m, lr), dtype=torch.bfloat16, device=d.device)
    _L.check(_L.lib().fp4x_hc_scaled_silu(_ptr(d), d.stride(0), _ptr(bot), m, lr, hc, _L.stream_of(d)),
             "hc_scaled_silu")
    return bot


def hc_gate_mean(normalized, g, hc):
    """block_input [M, H] from normalized [M, hc*H] and bf16 gate logits g [M, hc*H]."""
    _need_cuda(normalized, g)
    if normalized.stride(1) != 1:
        normalized = normalized.contiguous()
    if g.stride(1) != 1:
        g = g.contiguous()
    m, n = g.shape
    h = n // hc
    out = torch.empty((m, h), dtype=torch.bfloat16, device=g.device)
    _L.check(_L.lib().fp4x_hc_gate_mean(_ptr(normalized), normalized.stride(0), _ptr(g), g.stride(0), _ptr(out), m,
                                        h, hc, _L.stream_of(g)), "hc_gate_mean")
    return out


# ----------------------------------------------------------------- dequant
def mx8_dequant(w8, s_u8, rows=2048):
    """fp32 [N, K] = e4m3(w8) * 2^(s - 127) (HIP kernel)."""
    _need_cuda(w8, s_u8)
    n, k = w8.shape
    out = torch.empty((n, k), dtype=torch.float32, device=w8.device)
    _L.check(_L.lib().fp4x_mx8_dequant(_ptr(w8), _ptr(s_u8), n, k, _ptr(out), _L.stream_of(w8)), "mx8_dequant")
    return out


_FMT_BY_NAME = {"mx8": _L.FMT_MX8, "w8": _L.FMT_W8_F32, "w8_f16": _L.FMT_W8_F16, "w6": _L.FMT_W6,
                "nv4": _L.FMT_NV4, "int2": _L.FMT_INT2_F16, "int2_e4m3": _L.FMT_INT2_E4M3, "bf16": _L.FMT_BF16}


def dequant_operand(fmt, w0, w1=None, s=None, K=None, G=16):
    """The bf16 operand [N, K] the GEMV kernels decode from packed planes
    (same device decode functions as the GEMVs)."""
    _need_cuda(w0, w1, s)
    code = _FMT_BY_NAME[fmt]
    n = w0.shape[0]
    out = torch.empty((n, K), dtype=torch.bfloat16, device=w0.device)
    _L.check(_L.lib().fp4x_dequant_bf16(code, _ptr(w0), _ptr(w1), _ptr(s), n, K, G, _ptr(out), _L.stream_of(w0)),
             "dequant_bf16")
    return out


# ----------------------------------------------------------------- weight prep (torch)
ORDER = (0, 2, 1, 3)  # INT2: element j of each 4-group lives in bit pair ORDER[j]
_E2M1 = {}


# HIP weight preparation
_SRC_F32, _SRC_BF16, _SRC_MX8, _SRC_NV4 = 0, 1, 2, 3
_Q_W8, _Q_W6, _Q_NV4, _Q_INT2, _Q_INT2_E4M3 = 0, 1, 2, 3, 4


def _hip_src(w):
    """A dense fp32/bf16 device matrix as a HIP quantizer source, or None (CPU
    tensors and other dtypes take the torch formulas)."""
    if not isinstance(w, torch.Tensor) or not w.is_cuda or w.dim() != 2 or w.shape[1] % 64 \
            or w.dtype not in (torch.float32, torch.bfloat16):
        return None
    w = w.contiguous()
    return (_SRC_F32 if w.dtype == torch.float32 else _SRC_BF16, w, None, 0.0)


def _hip_quantize(src, n, k, dst, G=16, qmax=31, gs=0.0):
    """One fp4x_quantize call; returns the output planes of the target."""
    kind, a, b, sgs = src
    dev = a.device
    shapes = {_Q_W8: [(k, torch.int8), (k // 64, torch.float32)],
              _Q_W6: [(k // 2, torch.uint8), (k // 4, torch.uint8), (k // 32, torch.float16)],
              _Q_NV4: [(k // 2, torch.uint8), (k // 16, torch.float8_e4m3fn)],
              _Q_INT2: [(k // 4, torch.uint8), (k // G, torch.float16)],
              _Q_INT2_E4M3: [(k // 4, torch.uint8), (k // G, torch.float8_e4m3fn), (1, torch.float32)]}[dst]
    outs = [torch.empty((n, c), dtype=dt, device=dev) for c, dt in shapes]
    o = [_ptr(t) for t in outs] + [None] * (3 - len(outs))
    _L.check(_L.lib().fp4x_quantize(kind, _ptr(a), None if b is None else _ptr(b), float(sgs), n, k, dst, G, qmax,
                                    float(gs), o[0], o[1], o[2], _L.stream_of(a)), "quantize")
    return outs


def _hip_w6_clip(src, n, k, qmax, clip_search):
    """One fp4x_quantize_w6_clip call: (L, H, S)."""
    kind, a, b, sgs = src
    dev = a.device
    outs = [torch.empty((n, c), dtype=dt, device=dev)
            for c, dt in ((k // 2, torch.uint8), (k // 4, torch.uint8), (k // 32, torch.float16))]
    _L.check(_L.lib().fp4x_quantize_w6_clip(kind, _ptr(a), None if b is None else _ptr(b), float(sgs), n, k, qmax,
                                            clip_search, *[_ptr(t) for t in outs], _L.stream_of(a)), "quantize_w6_clip")
    return tuple(outs)


def _hip_nv4(src, n, k):
    """NVFP4 of a source: the global amax on the device (one host read, as the
    reference's .item()), gs = max(amax / 6 / 448, 1e-30), then the groups."""
    kind, a, b, sgs = src
    amax = torch.zeros(1, dtype=torch.float32, device=a.device)
    _L.check(_L.lib().fp4x_absmax(kind, _ptr(a), None if b is None else _ptr(b), float(sgs), n, k, _ptr(amax),
                                  _L.stream_of(a)), "absmax")
    gs = max(float(amax.item()) / 6.0 / 448.0, 1e-30)
    P, S = _hip_quantize(src, n, k, _Q_NV4, gs=gs)
    return P, S, gs


def requantize_mx8(w8, s_u8, fmt, group=16, qmax=31, clip_search=0, scale_fmt="fp16"):
    """quantize_<fmt>(mx8_dequant(w8, s_u8)) for fmt in w8, w6, nv4, int2, read
    from the packed MXFP8 rows without their fp32 copy (the plugin's layer and
    LM-head preparation, x/fp4patch.py:61-83, :357-359); clip_search for w6,
    scale_fmt for int2."""
    _need_cuda(w8, s_u8)
    n, k = w8.shape
    if k % 64 or (fmt == "int2" and group not in (16, 32, 64)) or clip_search > 64:
        wf = mx8_dequant(w8, s_u8)
        return {"w8": quantize_w8, "w6": lambda t: quantize_w6(t, qmax, clip_search), "nv4": quantize_nv4,
                "int2": lambda t: quantize_int2(t, scale_fmt, group)}[fmt](wf)
    src = (_SRC_MX8, w8.contiguous(), s_u8.contiguous().view(torch.uint8), 0.0)
    return _requantize(src, n, k, fmt, group, qmax, clip_search, scale_fmt)


def requantize_nv4(P, S, gs, fmt, group=16, qmax=31, scale_fmt="fp16"):
    """quantize_<fmt>(dequant_nv4(P, S, gs)) read from the packed NVFP4 rows
    without their fp32 copy (the draft head's INT2 copy, x/fp4patch.py:303-306);
    scale_fmt for int2."""
    _need_cuda(P, S)
    n, k = P.shape[0], P.shape[1] * 2
    if k % 64 or (fmt == "int2" and group not in (16, 32, 64)):
        wf = dequant_nv4(P, S, gs)
        return {"w8": quantize_w8, "w6": lambda t: quantize_w6(t, qmax), "nv4": quantize_nv4,
                "int2": lambda t: quantize_int2(t, scale_fmt, group)}[fmt](wf)
    src = (_SRC_NV4, P.contiguous(), S.contiguous().view(torch.uint8), float(gs))
    return _requantize(src, n, k, fmt, group, qmax, scale_fmt=scale_fmt)


def _requantize(src, n, k, fmt, group, qmax, clip_search=0, scale_fmt="fp16"):
    if fmt == "w8":
        return tuple(_hip_quantize(src, n, k, _Q_W8))
    if fmt == "w6" and clip_search:
        return _hip_w6_clip(src, n, k, qmax, clip_search)
    if fmt == "w6":
        return tuple(_hip_quantize(src, n, k, _Q_W6, qmax=qmax))
    if fmt == "nv4":
        return _hip_nv4(src, n, k)
    if fmt == "int2" and scale_fmt != "fp16":
        P, S, R = _hip_quantize(src, n, k, _Q_INT2_E4M3, G=group)
        return P, S, R.view(-1)
    if fmt == "int2":
        return tuple(_hip_quantize(src, n, k, _Q_INT2, G=group))
    raise ValueError(f"fp4x: unknown format {fmt!r}")


@torch.no_grad()
def quantize_w8(w):
    """Symmetric int8 with fp32 scales per 64: (q [N, K], s [N, K/64]).
    HIP kernel for device fp32/bf16 matrices, torch formulas otherwise."""
    src = _hip_src(w)
    if src is not None:
        return tuple(_hip_quantize(src, w.shape[0], w.shape[1], _Q_W8))
    n, k = w.shape
    g = w.float().reshape(n, k // 64, 64)
    s = g.abs().amax(-1).clamp_min(1e-12) / 127.0
    q = torch.round(g / s.unsqueeze(-1)).clamp(-127, 127).to(torch.int8).reshape(n, k)
    return q.contiguous(), s.contiguous()


def _w6_pack(codes):
    lo, hi = codes & 15, codes >> 4
    L = (lo[:, 0::2] | (lo[:, 1::2] << 4)).to(torch.uint8)
    H = (hi[:, 0::4] | (hi[:, 2::4] << 2) | (hi[:, 1::4] << 4) | (hi[:, 3::4] << 6)).to(torch.uint8)
    return L, H


@torch.no_grad()
def quantize_w6(w, qmax=31, clip_search=0):
    """W6 g32 two-plane layout: (L [N, K/2], H [N, K/4], S fp16 [N, K/32]).
    qmax < 31 quantizes to fewer levels in the same layout.  HIP kernels for
    device fp32/bf16 matrices (the clip search for up to 64 clip factors)."""
    src = _hip_src(w)
    if src is not None and not clip_search:
        return tuple(_hip_quantize(src, w.shape[0], w.shape[1], _Q_W6, qmax=qmax))
    if src is not None and 0 < clip_search <= 64:
        return _hip_w6_clip(src, w.shape[0], w.shape[1], qmax, clip_search)
    n, k = w.shape
    L = torch.empty((n, k // 2), dtype=torch.uint8, device=w.device)
    H = torch.empty((n, k // 4), dtype=torch.uint8, device=w.device)
    S = torch.empty((n, k // 32), dtype=torch.float16, device=w.device)
    for r0 in range(0, n, 2048):
        g = w[r0:r0 + 2048].float().reshape(-1, k // 32, 32)
        s = (g.abs().amax(-1, keepdim=True) / qmax).to(torch.float16).float().clamp_min(6.2e-5)
        if clip_search:
            def sq_err(sc):
                return ((torch.round(g / sc).clamp(-qmax - 1, qmax) * sc - g) ** 2).sum(-1, keepdim=True)
            best, bs = sq_err(s), s
            for c in torch.linspace(0.70, 0.98, clip_search).tolist():
                sc = (s * c).to(torch.float16).float().clamp_min(6.2e-5)
                e = sq_err(sc)
                better = e < best
                best = torch.where(better, e, best)
                bs = torch.where(better, sc, bs)
            s = bs
        codes = (torch.round(g / s).clamp(-qmax - 1, qmax).to(torch.int32) + 32).reshape(-1, k)
        L[r0:r0 + 2048], H[r0:r0 + 2048] = _w6_pack(codes)
        S[r0:r0 + 2048] = s.squeeze(-1).to(torch.float16)
    return L, H, S


@torch.no_grad()
def quantize_nv4(w, rows=2048):
    """RTN NVFP4: (P [N, K/2] e2m1 pairs, S [N, K/16] e4m3, gs python float).
    HIP kernels for device fp32/bf16 matrices."""
    src = _hip_src(w)
    if src is not None:
        return _hip_nv4(src, w.shape[0], w.shape[1])
    n, k = w.shape
    lut = _E2M1.get(w.device)
    if lut is None:
        lut = _E2M1[w.device] = torch.tensor([0, .5, 1, 1.5, 2, 3, 4, 6], device=w.device)
    amax = 0.0
    for r0 in range(0, n, rows):
        amax = max(amax, w[r0:r0 + rows].float().abs().max().item())
    gs = max(amax / 6.0 / 448.0, 1e-30)
    mids = (lut[1:] + lut[:-1]) / 2
    P = torch.empty((n, k // 2), dtype=torch.uint8, device=w.device)
    S = torch.empty((n, k // 16), dtype=torch.float8_e4m3fn, device=w.device)
    for r0 in range(0, n, rows):
        g = w[r0:r0 + rows].float().reshape(-1, k // 16, 16)
        sc = (g.abs().amax(-1, keepdim=True) / 6.0 / gs).clamp(min=2 ** -9, max=448.0).to(torch.float8_e4m3fn)
        v = (g / (sc.float() * gs)).clamp(-6, 6)
        code = (torch.bucketize(v.abs(), mids) | ((v < 0).to(torch.int64) << 3)).reshape(-1, k)
        P[r0:r0 + rows] = (code[:, 0::2] | (code[:, 1::2] << 4)).to(torch.uint8)
        S[r0:r0 + rows] = sc.reshape(-1, k // 16)
    return P, S, gs


@torch.no_grad()
def quantize_int2(weight, scale_fmt="fp16", group=16):
    """INT2 per group (levels -1.5..1.5 x s): fp16 -> (P, S); e4m3 -> (P, S_e4m3, row_scale fp32).
    HIP kernels for device fp32/bf16 matrices and G = 16, 32, 64 (any scale_fmt
    other than "fp16" is the e4m3 form, as in the reference)."""
    src = _hip_src(weight)
    if src is not None and group in (16, 32, 64):
        if scale_fmt == "fp16":
            return tuple(_hip_quantize(src, weight.shape[0], weight.shape[1], _Q_INT2, G=group))
        P, S, R = _hip_quantize(src, weight.shape[0], weight.shape[1], _Q_INT2_E4M3, G=group)
        return P, S, R.view(-1)
    n, k = weight.shape
    P = torch.empty((n, k // 4), dtype=torch.uint8, device=weight.device)
    S = torch.empty((n, k // group), dtype=torch.float16 if scale_fmt == "fp16" else torch.float8_e4m3fn,
                    device=weight.device)
    R = torch.empty((n,), dtype=torch.float32, device=weight.device)
    for r0 in range(0, n, 8192):
        g = weight[r0:r0 + 8192].float().reshape(-1, k // group, group)
        s = g.abs().amax(-1, keepdim=True).clamp_min(1e-8) / 1.5
        if scale_fmt == "fp16":
            s = s.half()
            sf = s.float()
        else:
            rs = s.amax(1, keepdim=True) / 448.0
            s = (s / rs).to(torch.float8_e4m3fn)
            sf = s.float() * rs
            R[r0:r0 + 8192] = rs.reshape(-1)
        code = (torch.floor(g / sf) + 2).clamp(0, 3).to(torch.uint8).reshape(-1, k // 4, 4)
        b = torch.zeros(code.shape[:2], dtype=torch.uint8, device=weight.device)
        for j in range(4):
            b |= code[..., j] << (2 * ORDER[j])
        P[r0:r0 + 8192] = b
        S[r0:r0 + 8192] = s.squeeze(-1)
    return (P, S) if scale_fmt == "fp16" else (P, S, R)


def dequant_int2(packed, scales):
    """fp32 [N, K] = (code - 1.5) * s per group."""
    n = packed.shape[0]
    k = packed.shape[1] * 4
    code = torch.stack([(packed >> (2 * ORDER[j])) & 3 for j in range(4)], -1).reshape(n, k).float() - 1.5
    g = k // scales.shape[1]
    return (code.reshape(n, k // g, g) * scales.float().unsqueeze(-1)).reshape(n, k)


@torch.no_grad()
def dequant_nv4(P, S, gs):
    """fp32 [N, K] = e2m1(P) * e4m3(S) * gs."""
    lut = torch.tensor([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], device=P.device)
    n = P.shape[0]
    v = torch.stack([lut[(P & 15).long()], lut[(P >> 4).long()]], -1).reshape(n, -1)
    return (v.reshape(n, -1, 16) * S.float().unsqueeze(-1) * gs).reshape(n, -1)


@torch.no_grad()
def quantize_mx8(w):
    """OCP Microscaling MXFP8: e4m3 elements with an e8m0 exponent per 32
    (shared exponent floor(log2(amax)) - 8, clamped to [-127, 127]; elements
    rounded to nearest even, saturating at +-448).  Returns (w uint8 [N, K],
    s uint8 [N, K/32]).  The plugin receives MXFP8 weights pre-packed; this is
    the packer for synthetic and converted weights."""
    n, k = w.shape
    g = w.float().reshape(n, k // 32, 32)
    amax = g.abs().amax(-1)
    e = ((amax.view(torch.int32) >> 23) & 0xFF) - 127
    e = torch.where(amax.view(torch.int32) >> 23 == 0, torch.full_like(e, -135), e)
    X = (e - 8).clamp(-127, 127)
    scaled = (g.double() / torch.exp2(X.double()).unsqueeze(-1)).float().clamp(-448.0, 448.0)
    q = scaled.to(torch.float8_e4m3fn).view(torch.uint8).reshape(n, k)
    return q.contiguous(), (X + 127).to(torch.uint8).contiguous()
