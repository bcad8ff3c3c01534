"""Benchmark of the fp4x decode GEMVs on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--kernels all|none|A,B,...]

Headline (one JSON line): the int8 g64 router-gate GEMV of a decode step —
48 independent [512 x 2560] gates at M = 3 (1 target + 2 draft rows), one
fp16 scale per 64 K values, fp32 logits — as one layer-batched launch.  A step is one such launch
over one batch of synthetic input; `value` is algorithmic bytes (weights +
scales + activations + logits) per second with all inputs resident in HBM.
Weights rotate through copies totalling > 512 MB so every launch streams from
HBM rather than the 256 MB MALL.

Why the gates carry the headline: the metric is quoted per kernel at decode
M, the MXFP8 GEMV is the workload the reference's own CPU path runs, and the
router-gate launch is the next one named, which fits one GPU; so it is the
headline, and every other workload (MXFP8, W6 and NVFP4 at M = 1/3/16, the
mixer, the 240 MB INT2 head) is a row of `kernels` with its own fraction of
peak and of the measured read ceiling.

`kernels` adds per-kernel µs and GB/s for every configuration (MXFP8 4096 x
2560, W6 8192 x 2560, NVFP4 16384 x 2560 at M = 1/3/16, single router gates
and the 48-gate launch with fp16 and with the reference's fp32 scales, the
97-layer mixer at the synthetic and the served shape, the 248,320-row fast
LM head and the exact MXFP8 head it replaces, the 65k-token draft head),
timed as HIP-graph replays, and the load-time weight preparation (group G,
eager), the MTP layer's int8 linears (H), and the served model's dense
linears at M = 3 in W6 and MXFP8 (I).  `read_ceiling` times a plain coalesced read of each kernel's bytes
under the same protocol (the fastest of a sweep of load depths and grids);
each kernel row carries `frac_of_ceiling`, that read's time over the
kernel's.  `cpu_baseline` times the reference math as PyTorch CPU ops
(oracle/torch_cpu.py) on the host cores for every configuration, with and
without the dequantization, and the fast head's selection and argmax against
the oracle on a sample of full-size rows.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "qwen3.8-flash-next-fp4-local-spark_amd")
sys.path[:0] = [ROOT, PKG]

PEAK_GBS = 8000.0
MALL_COLD_BYTES = 512 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--kernels", default="all", help="all | none | comma list of A,B,C,D,E,F,G,H,I")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-ceiling", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (--steps times): the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    return ap.parse_args()


def calibrate_copy(mib, steps):
    import torch
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": steps}), flush=True)


# ------------------------------------------------------------------ timing
def graph_time(fn_list, replays=20):
    """Average µs per call of the callables in fn_list, captured in one HIP
    graph (back to back, one call each) and replayed; events on the stream."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in fn_list[:2]:
            f()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for f in fn_list:
                f()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(replays):
            g.replay()
        e1.record(s)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (replays * len(fn_list))


def copies_for(nbytes):
    return max(2, -(-MALL_COLD_BYTES // max(nbytes, 1)))


def entry(us, nbytes):
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"us": round(us, 3), "bytes": int(nbytes), "GBps": round(gbs, 1), "frac_peak": round(gbs / PEAK_GBS, 4)}


# ------------------------------------------------------------------ workloads
def w8_f16(torch, w):
    """Symmetric int8 with one fp16 scale per 64 K values (last dim): the
    scale is amax / 127 rounded to fp16, and q = round(w / s) against it."""
    grp = w.reshape(*w.shape[:-1], w.shape[-1] // 64, 64)
    s16 = (grp.abs().amax(-1).clamp_min(1e-12) / 127.0).half()
    q = torch.round(grp / s16.float().unsqueeze(-1)).clamp(-127, 127).to(torch.int8).reshape(w.shape)
    return q.contiguous(), s16.contiguous()


def gate_weights(F, torch, dev, layers=48, n=512, k=2560, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    return w8_f16(torch, torch.randn((layers, n, k), generator=g, device=dev) * 0.02)


def gate_bytes(layers, M, n, k, s_bytes=2, out_bytes=4):
    return layers * (n * k + n * (k // 64) * s_bytes + M * k * 2 + M * n * out_bytes)


def bench_dense(F, torch, dev, out):
    import numpy as np
    cfgs = [("A_mx8_4096x2560", "mx8", 4096, 2560), ("C_w6_8192x2560", "w6", 8192, 2560),
            ("C_nv4_16384x2560", "nv4", 16384, 2560)]
    for name, fmt, n, k in cfgs:
        g = torch.Generator(device=dev).manual_seed(0)
        w = torch.randn((n, k), generator=g, device=dev) * 0.02
        if fmt == "mx8":
            planes = F.quantize_mx8(w)
            wbytes = n * k + n * k // 32
            fn = lambda x, p: F.mx8_linear(x, *p, (32, 512, 1, 4))
        elif fmt == "w6":
            planes = F.quantize_w6(w)
            wbytes = n * k // 2 + n * k // 4 + n * (k // 32) * 2
            fn = lambda x, p: F.w6_linear(x, *p, (32, 256, 1, 4))
        else:
            P, S, gs = F.quantize_nv4(w)
            planes = (P, S, gs)
            wbytes = n * k // 2 + n * (k // 16) + 4
            fn = lambda x, p: F.nv4_linear(x, *p, (32, 256, 4))
        ncp = copies_for(wbytes)
        copies = [tuple(t.clone() if torch.is_tensor(t) else t for t in planes) for _ in range(ncp)]
        for M in (1, 3, 16):
            x = torch.randn((M, k), generator=g, device=dev).to(torch.bfloat16)
            us = graph_time([lambda p=p: fn(x, p) for p in copies] * 2)
            out[f"{name}_M{M}"] = entry(us, wbytes + M * k * 2 + M * n * 2)
        del copies, planes, w
        torch.cuda.empty_cache()


def bench_mtp(F, torch, dev, out):
    """The MTP layer's linears as FP4X_MTP_W8=1 serves them (int8 g64 copies of its bf16 weights, fp32
    scales, bf16 out, the plugin's CFG_W8 K split or one slice): attention qkv [13312 x 2560], output
    [2560 x 6144], shared-expert gate/up [1280 x 2560] and down [2560 x 640] (the shapes the reference's
    MTP weight patch names, x/fp4patch.py:513-525), at M = 3 (1 target + 2 draft rows).  Its router gate
    [512 x 2560] and its mixers take the B and D rows' kernels."""
    import fp4patch
    for n, k in ((13312, 2560), (2560, 6144), (1280, 2560), (2560, 640)):
        g = torch.Generator(device=dev).manual_seed(7)
        q, s = F.quantize_w8(torch.randn((n, k), generator=g, device=dev) * 0.02)
        cfg = fp4patch.CFG_W8.get((n, k)) or (32, fp4patch._k_tile(k, (256, 64)), 1, 4)
        wbytes = n * k + n * (k // 64) * 4
        copies = [(q.clone(), s.clone()) for _ in range(copies_for(wbytes))]
        x = torch.randn((3, k), generator=g, device=dev).to(torch.bfloat16)
        us = graph_time([lambda c=c: F.w8_linear(x, c[0], c[1], cfg) for c in copies] * 2)
        out[f"H_mtp_w8_{n}x{k}_M3"] = entry(us, wbytes + 3 * k * 2 + 3 * n * 2)
        del copies, q, s
        torch.cuda.empty_cache()


def bench_shapes(F, torch, dev, out):
    """The served model's dense linears as the plugin calls them: every (N, K)
    of its tile tables (x/fp4patch.py:11-18) at M = 3 (1 target + 2 draft
    rows), in W6 (the shipped FP4X_DENSE=w6, CFG_W6's K split) and in MXFP8
    (the plugin's default dense mode, _mx8_cfg), bf16 out, the attention
    output projection [2560 x 6144] at M = 1 as well; weights rotate from
    HBM."""
    import fp4patch
    shapes = sorted(set(fp4patch.CFG_W6) | set(fp4patch.CFG_MX8))
    for fmt in ("w6", "mx8"):
        for n, k in shapes:
            g = torch.Generator(device=dev).manual_seed(11)
            w = torch.randn((n, k), generator=g, device=dev) * 0.02
            if fmt == "w6":
                planes = F.quantize_w6(w)
                wbytes = n * k // 2 + n * k // 4 + n * (k // 32) * 2
                cfg = fp4patch.CFG_W6.get((n, k)) or (32, 256, 1, 4)
                fn = lambda x, p, cfg=cfg: F.w6_linear(x, *p, cfg)
            else:
                planes = F.quantize_mx8(w)
                wbytes = n * k + n * (k // 32)
                cfg = fp4patch._mx8_cfg(n, k)
                fn = lambda x, p, cfg=cfg: F.mx8_linear(x, *p, cfg)
            copies = [tuple(t.clone() for t in planes) for _ in range(copies_for(wbytes))]
            for M in ((1, 3) if (n, k) == (2560, 6144) else (3,)):
                x = torch.randn((M, k), generator=g, device=dev).to(torch.bfloat16)
                us = graph_time([lambda p=p: fn(x, p) for p in copies] * 2)
                out[f"I_{fmt}_{n}x{k}_M{M}"] = entry(us, wbytes + M * k * 2 + M * n * 2)
            del copies, planes, w
            torch.cuda.empty_cache()


def bench_gates_single(F, torch, dev, out, q, s):
    """One router gate per launch, as the plugin calls them (x/fp4patch.py:264-272):
    the 48 gates back to back from HBM (copies rotating past the MALL), fp16
    scales and the reference's fp32 scales; and the 48-gate layer-batched
    launch with fp32 scales."""
    M, n, k = 3, 512, 2560
    L = q.shape[0]
    x = torch.randn((M, k), device=dev).to(torch.bfloat16)
    s32 = s.float()
    for name, ss, sb in (("B_w8_gate_single_layer_M3", s, 2), ("B_w8_gate_single_layer_M3_f32s", s32, 4)):
        # the graph cycles through copies of the 48 gates spanning more than
        # the MALL, so every gate streams from HBM; the MALL-warm figure (the
        # 48 gates alone, 63 MB, replayed) is kept beside it
        ncp = copies_for(L * (n * k + n * (k // 64) * sb))
        cps = [(q.clone(), ss.clone()) for _ in range(ncp - 1)] + [(q, ss)]
        calls = [lambda c=c, i=i: F.w8_linear(x, c[0][i], c[1][i], (16, 512, 1, 4), torch.float32)
                 for c in cps for i in range(L)]
        out[name] = entry(graph_time(calls, 5), gate_bytes(1, M, n, k, s_bytes=sb))
        warm = [lambda i=i: F.w8_linear(x, q[i], ss[i], (16, 512, 1, 4), torch.float32) for i in range(L)]
        out[name]["us_mall_warm"] = round(graph_time(warm), 3)
        del cps
    b32 = gate_bytes(L, M, n, k, s_bytes=4)
    ncp = copies_for(L * (n * k + n * (k // 64) * 4))
    qs = [(q.clone(), s32.clone()) for _ in range(ncp - 1)] + [(q, s32)]
    x3 = torch.randn((L, M, k), device=dev).to(torch.bfloat16)
    us = graph_time([lambda c=c: F.w8_linear_layers(x3, c[0], c[1], torch.float32) for c in qs] * 2)
    out["B_w8_gates_48_layers_M3_f32s"] = entry(us, b32)
    del qs


def mixer_bytes(M, nd, lr, hc, H, s_bytes):
    down = nd * hc * H + nd * (hc * H // 64) * s_bytes + M * hc * H * 2 + M * nd * 2 + M * lr * 2
    up = hc * H * lr + hc * H * (lr // 64) * s_bytes + M * lr * 2 + M * hc * H * 2 + M * H * 2
    return down, up


def bench_hc(F, torch, dev, out, layers=97):
    """97 mixers back to back: the synthetic shape (down [640 x 10240], up
    [10240 x 640], 16 K slices) with fp16 scales (as two launches and as one)
    and with the reference's fp32 scales; the served shape (down [336 x
    10240], up [10240 x 320], 8 K slices, fp32 scales: the plugin's fused
    mixer, x/fp4patch.py:201-220)."""
    HC, H, M = 4, 2560, 3
    g = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn((M, HC * H), generator=g, device=dev).to(torch.bfloat16)

    def layers_of(nd, lr, f16):
        mix = []
        for _ in range(layers):
            wd = torch.randn((nd, HC * H), generator=g, device=dev) * 0.02
            wu = torch.randn((HC * H, lr), generator=g, device=dev) * 0.02
            qd, sd = w8_f16(torch, wd) if f16 else F.quantize_w8(wd)
            qu, su = w8_f16(torch, wu) if f16 else F.quantize_w8(wu)
            qi, si = F.HCFused.interleave_up(qu, su, HC, 8)
            mix.append((qd, sd, qi, si))
        return mix

    # synthetic shape, fp16 scales: down, up, the pair as two launches, one launch
    ND, LR, KS = 640, 640, 16
    fx = F.HCFused(dev, n_down=ND, max_ksplit=KS)
    mix = layers_of(ND, LR, True)
    down_b, up_b = mixer_bytes(M, ND, LR, HC, H, 2)
    bots = [fx.down(x, qd, sd, LR, HC, (32, 256, KS, 4))[1] for qd, sd, _, _ in mix]
    us_down = graph_time([lambda m=m: fx.down(x, m[0], m[1], LR, HC, (32, 256, KS, 4)) for m in mix], replays=5)
    us_up = graph_time([lambda m=m, b=b: F.HCFused.up(b, m[2], m[3], x, HC, (8, 64, 4)) for m, b in zip(mix, bots)],
                       replays=5)

    def both(m):
        _, bot = fx.down(x, m[0], m[1], LR, HC, (32, 256, KS, 4))
        F.HCFused.up(bot, m[2], m[3], x, HC, (8, 64, 4))
    us_pair = graph_time([lambda m=m: both(m) for m in mix], replays=5)
    us_mix = graph_time([lambda m=m: fx.mix(x, m[0], m[1], LR, HC, m[2], m[3], x, (32, 256, KS, 4)) for m in mix],
                        replays=5)
    out["D_hc_down_640x10240_M3"] = entry(us_down, down_b)
    out["D_hc_up_10240x640_M3"] = entry(us_up, up_b)
    out["D_hc_mixer_97_layers_M3"] = dict(entry(us_pair * layers, (down_b + up_b) * layers),
                                          us_per_mixer=round(us_pair, 3))
    out["D_hc_mix_one_call_97_layers_M3"] = dict(entry(us_mix * layers, (down_b + up_b) * layers),
                                                 us_per_mixer=round(us_mix, 3))
    del mix, bots
    # synthetic shape, fp32 scales (the reference's quantize_w8 layout)
    mix = layers_of(ND, LR, False)
    down_b, up_b = mixer_bytes(M, ND, LR, HC, H, 4)
    us_mix = graph_time([lambda m=m: fx.mix(x, m[0], m[1], LR, HC, m[2], m[3], x, (32, 256, KS, 4)) for m in mix],
                        replays=5)
    out["D_hc_mix_one_call_97_layers_M3_f32s"] = dict(entry(us_mix * layers, (down_b + up_b) * layers),
                                                      us_per_mixer=round(us_mix, 3))
    del mix
    # the served shape, fp32 scales, 8 K slices
    ND, LR, KS = 336, 320, 8
    fx = F.HCFused(dev)
    mix = layers_of(ND, LR, False)
    down_b, up_b = mixer_bytes(M, ND, LR, HC, H, 4)
    us_mix = graph_time([lambda m=m: fx.mix(x, m[0], m[1], LR, HC, m[2], m[3], x, (32, 256, KS, 4)) for m in mix],
                        replays=5)
    out["D_hc_mix_served_336x10240_10240x320_97_layers_M3_f32s"] = dict(
        entry(us_mix * layers, (down_b + up_b) * layers), us_per_mixer=round(us_mix, 3))
    del mix


def bench_head(F, torch, dev, out, vectors=1000, n_x=128):
    """The fast target head at V = 248,320, K = 2560, M = 3, G = 16, C = 512.
    The coarse pass rotates three INT2 copies (720 MB); the refine and the
    whole head rotate n_x activation sets, so the 3 x 512 MXFP8 rows each call
    gathers (4 MB) differ from call to call and come from HBM, not the MALL.
    Returns the head's tensors for the CPU leg's parity check."""
    V, K, C, M = 248320, 2560, 512, 3
    g = torch.Generator(device=dev).manual_seed(2)
    w = torch.randn((V, K), generator=g, device=dev) * 0.02
    rows = torch.randperm(V, generator=g, device=dev)[:64]
    w[rows] *= 4
    q, s = F.quantize_mx8(w)
    del w
    P, S = F.quantize_int2(F.mx8_dequant(q, s), group=16)
    torch.cuda.empty_cache()
    int2_b = V * K // 4 + V * (K // 16) * 2 + M * K * 2 + M * V * 2
    copies = [(P.clone(), S.clone()) for _ in range(2)] + [(P, S)]
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    us = graph_time([lambda c=c: F.int2_logits(x, c[0], c[1], V, out_dtype=torch.bfloat16) for c in copies], 10)
    out["E_int2_coarse_248320x2560_M3"] = entry(us, int2_b)
    # the variant with e4m3 group scales and an fp32 scale per row, on the same streaming kernel as the
    # fp16-scaled head (its e4m3 instance); its copy from the device quantizer, three copies rotated
    wf = F.mx8_dequant(q, s)
    P8, S8, R8 = F.quantize_int2(wf, scale_fmt="e4m3", group=16)
    del wf
    torch.cuda.empty_cache()
    copies8 = [(P8.clone(), S8.clone(), R8.clone()) for _ in range(2)] + [(P8, S8, R8)]
    us = graph_time([lambda c=c: F.int2_logits(x, c[0], c[1], V, RS=c[2], out_dtype=torch.bfloat16)
                     for c in copies8], 10)
    out["E_int2_e4m3_rowscale_coarse_248320x2560_M3"] = entry(us, V * K // 4 + V * (K // 16) + V * 4 + M * K * 2 +
                                                               M * V * 2)
    del copies8, P8, S8, R8
    torch.cuda.empty_cache()
    # fp16 scales per 32 K values (the plugin's FP4X_HEAD_G=32): 16% fewer bytes, the same streaming kernel
    wf = F.mx8_dequant(q, s)
    P32, S32 = F.quantize_int2(wf, group=32)
    del wf
    torch.cuda.empty_cache()
    copies32 = [(P32.clone(), S32.clone()) for _ in range(2)] + [(P32, S32)]
    us = graph_time([lambda c=c: F.int2_logits(x, c[0], c[1], V, out_dtype=torch.bfloat16) for c in copies32], 10)
    out["E_int2_g32_coarse_248320x2560_M3"] = entry(us, V * K // 4 + V * (K // 32) * 2 + M * K * 2 + M * V * 2)
    # ... with the top-1024 set the reference pairs with G = 32 (x/fp4patch.py:345)
    us = graph_time([lambda c=c: F.int2_topk(x, c[0], c[1], V, 1024, sorted=False) for c in copies32], 10)
    out["E_int2_g32_coarse_plus_top1024_set_M3"] = {"us": round(us, 3)}
    del copies32, P32, S32
    torch.cuda.empty_cache()
    # the top-C alone over 16 coarse outputs of different activations, one graph
    coarses = [F.int2_logits(torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16), P, S, V,
                             out_dtype=torch.bfloat16) for _ in range(16)]
    us = graph_time([lambda co=co: F.topk_rows(co, C) for co in coarses], 10)
    out["E_topk512_M3"] = dict(entry(us, M * V * 2 + M * C * 8), coarse_sets=len(coarses))
    del coarses
    # the coarse pass and the top-C in one call (slice maxima from the coarse kernel);
    # the fast head asks for the set only (it scatters exact logits at the indices)
    us = graph_time([lambda c=c: F.int2_topk(x, c[0], c[1], V, C) for c in copies], 10)
    out["E_int2_coarse_plus_topk512_M3"] = entry(us, int2_b + M * C * 8)
    us = graph_time([lambda c=c: F.int2_topk(x, c[0], c[1], V, C, sorted=False) for c in copies], 10)
    out["E_int2_coarse_plus_top512_set_M3"] = entry(us, int2_b + M * C * 8)
    # the exact rescore of 3 x 512 candidate rows, over n_x activation sets and their candidates
    xs = [torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16) for _ in range(n_x)]
    pairs = [F.int2_topk(xx, P, S, V, C, sorted=False) for xx in xs]
    ref_b = M * C * (K + K // 32 + 8) + M * K * 2 + M * C * 2
    us = graph_time([lambda i=i: F.refine_mx8_(pairs[i][0], xs[i], pairs[i][1], q, s) for i in range(n_x)], 5)
    out["E_refine_mx8_3x512_M3"] = dict(entry(us, ref_b), activation_sets=n_x)

    def head(xx, c):
        co, ix = F.int2_topk(xx, c[0], c[1], V, C, sorted=False)
        F.refine_mx8_(co, xx, ix, q, s)
    us = graph_time([lambda i=i: head(xs[i], copies[i % 3]) for i in range(n_x)], 3)
    out["E_fast_head_total_M3"] = {"us": round(us, 3), "activation_sets": n_x}
    del pairs
    # the exact head the fast path replaces: the MXFP8 GEMV over all 248,320 rows
    # (655 MB, above the 256 MB MALL, so one copy streams from HBM)
    us = graph_time([lambda: F.mx8_linear(x, q, s, (32, 512, 1, 4))] * 2, 10)
    out["E_exact_head_mx8_248320x2560_M3"] = entry(us, V * K + V * K // 32 + M * K * 2 + M * V * 2)
    # argmax agreement against the exact-weight MXFP8 GEMV over seeded vectors (the CPU leg compares the
    # same argmaxes with the oracle's fast head)
    agree, n, x_rows, fast_am = 0, 0, [], []
    for b0 in range(1000, 1000 + vectors, M):
        rng = torch.Generator(device=dev).manual_seed(b0)
        xs_ = torch.randn((M, K), generator=rng, device=dev).to(torch.bfloat16)
        co, ix = F.int2_topk(xs_, P, S, V, C, sorted=False)
        fast = F.refine_mx8_(co, xs_, ix, q, s)
        full = F.mx8_linear(xs_, q, s, (32, 512, 1, 4))
        m = min(M, 1000 + vectors - b0)
        agree += int((fast[:m].argmax(-1) == full[:m].argmax(-1)).sum())
        n += m
        x_rows.append(xs_[:m].view(torch.int16).cpu())
        fast_am.append(fast[:m].argmax(-1).cpu())
    out["E_fast_head_total_M3"]["argmax_agreement"] = round(agree / n, 4)
    out["E_fast_head_total_M3"]["vectors"] = n
    del copies, xs
    return q, s, P, S, (torch.cat(x_rows), torch.cat(fast_am))


# ------------------------------------------------------------------ CPU baseline
def bench_draft(F, torch, dev, out):
    """The MTP draft head over a 65,197-token subset of a 248,320-token NVFP4
    head (x/fp4patch.py:279-334): INT2 coarse + top-64 + exact NVFP4 rescore,
    and the NVFP4 GEMV over the whole subset."""
    sys.path.insert(0, os.path.join(ROOT, "qwen3.8-flash-next-fp4-local-spark_amd"))
    import fp4patch
    V, K, M, NS, DC = 248320, 2560, 3, 65197, 64
    g = torch.Generator(device=dev).manual_seed(4)
    P = torch.randint(0, 256, (V, K // 2), generator=g, device=dev, dtype=torch.uint8)
    S = (torch.randint(0x28, 0x40, (V, K // 16), generator=g, device=dev, dtype=torch.uint8)).view(torch.float8_e4m3fn)
    ids = torch.sort(torch.randperm(V, generator=g, device=dev)[:NS]).values
    st = fp4patch._draft_prepare(F, P, S, 1.0e-3, ids, DC)
    del P, S
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    int2_b = NS * (K // 4) + NS * (K // 16) * 2 + M * K * 2
    ncp = copies_for(int2_b)
    copies = [dict(st, c=(st["c"][0].clone(), st["c"][1].clone())) for _ in range(ncp)]
    us = graph_time([lambda c=c: fp4patch._draft_logits(F, x, c, V, DC) for c in copies], 10)
    out["F_draft_head_65k_int2_top64_nv4_M3"] = entry(us, int2_b + M * DC * (K // 2 + K // 16 + 8) + M * V * 2)
    # the exact rescore alone, over n_x activation sets and their own candidates
    # (rows not read by the previous call), one graph
    n_x = 64
    xs = [torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16) for _ in range(n_x)]
    cands = [F.int2_topk(xx, *st["c"], NS, DC, sorted=False)[1] for xx in xs]
    us = graph_time([lambda i=i: F.refine_nv4(xs[i], cands[i], st["w"], st["s"], st["gs"]) for i in range(n_x)], 5)
    out["F_refine_nv4_3x64_M3"] = dict(entry(us, M * DC * (K // 2 + K // 16 + 8) + M * K * 2 + M * DC * 4),
                                       activation_sets=n_x)
    del xs, cands
    nv4_b = NS * (K // 2 + K // 16) + M * K * 2 + M * NS * 2
    ncp = copies_for(nv4_b)
    wc = [(st["w"].clone(), st["s"].clone()) for _ in range(ncp)]
    us = graph_time([lambda c=c: F.nv4_linear(x, c[0], c[1], st["gs"], (32, 256, 4)) for c in wc], 10)
    out["F_draft_subset_nv4_65197x2560_M3"] = entry(us, nv4_b)
    del copies, wc, st


def bench_prep(F, torch, dev, out):
    """Weight preparation (x/fp4patch.py:61-83, :179-182, :357-359), eager as the
    plugin runs it at load: the LM head's INT2 copy and a dense layer's NVFP4
    and W6 copies straight from packed MXFP8 rows, and the mixer's W8 copy of a
    bf16 weight.  Bytes: packed source read + packed output written."""
    g = torch.Generator(device=dev).manual_seed(9)

    def timed(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    V, K = 248320, 2560
    q, s = F.quantize_mx8(torch.randn((V, K), generator=g, device=dev) * 0.02)
    torch.cuda.empty_cache()
    us = timed(lambda: F.requantize_mx8(q, s, "int2", group=16))
    out["G_prep_int2_from_mx8_248320x2560"] = dict(entry(us, V * K + V * K // 32 + V * K // 4 + V * K // 16 * 2),
                                                   fp32_copy_avoided_MB=round(V * K * 4 / 1e6))
    del q, s
    N = 16384
    q, s = F.quantize_mx8(torch.randn((N, K), generator=g, device=dev) * 0.02)
    src = N * K + N * K // 32
    us = timed(lambda: F.requantize_mx8(q, s, "nv4"))
    out["G_prep_nv4_from_mx8_16384x2560"] = entry(us, src + N * K // 2 + N * K // 16)
    us = timed(lambda: F.requantize_mx8(q, s, "w6"))
    out["G_prep_w6_from_mx8_16384x2560"] = entry(us, src + N * K // 2 + N * K // 4 + N * K // 32 * 2)
    w = (torch.randn((336, 10240), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    us = timed(lambda: F.quantize_w8(w))
    out["G_prep_w8_from_bf16_336x10240"] = entry(us, 336 * 10240 * 2 + 336 * 10240 + 336 * 160 * 4)
    del q, s, w


# ------------------------------------------------------------------ read ceiling
def bench_read_ceiling(F, torch, dev, sizes, replays=10):
    """{bytes: (µs, shape)}: the fastest plain coalesced read (fp4x_read_ceiling)
    of each size, timed as the kernels are: graph replays back to back, the
    source rotating over > 512 MB so every read streams from HBM; swept over
    4/8/16 loads in flight and 2/4/8 workgroups per CU."""
    import ctypes
    lib = F._L.lib()
    total = 640 << 20
    buf = torch.ones(total, dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    base = buf.data_ptr()
    res = {}
    for nbytes in sorted(set(sizes)):
        b16 = -(-nbytes // 16) * 16
        if b16 > total // 2:
            continue
        span = -(-b16 // 4096) * 4096
        ncp = max(2, min(total // span, -(-MALL_COLD_BYTES // span)))
        best = None
        for unroll in (4, 8, 16):
            for wpc in (2, 4, 8):
                def call(off, unroll=unroll, wpc=wpc):
                    F._L.check(lib.fp4x_read_ceiling(ctypes.c_void_p(base + off), b16, unroll, wpc, F._ptr(sink),
                                                     F._L.stream_of(buf)), "read_ceiling")
                us = graph_time([lambda o=i * span: call(o) for i in range(ncp)], replays)
                if best is None or us < best[0]:
                    best = (us, f"{unroll} loads in flight x {wpc} WG/CU")
        res[nbytes] = best
    del buf
    torch.cuda.empty_cache()
    return res


def attach_ceilings(kernels, ceil):
    """frac_of_ceiling = plain-read µs / kernel µs for each kernel row (per
    mixer for the 97-layer rows)."""
    for row in kernels.values():
        if "bytes" not in row:
            continue
        nb, us = row["bytes"], row["us"]
        if "us_per_mixer" in row:
            nb, us = nb // 97, row["us_per_mixer"]
        c = ceil.get(nb)
        if c:
            row["read_ceiling_us"] = round(c[0], 3)
            row["frac_of_ceiling"] = round(c[0] / us, 4)


def ceiling_sizes(kernels):
    out = []
    for row in kernels.values():
        if "bytes" in row:
            out.append(row["bytes"] // 97 if "us_per_mixer" in row else row["bytes"])
    return out


# ------------------------------------------------------------------ CPU baseline
def _median_us(fn, reps, warm=3):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter_ns()
        fn()
        ts.append(time.perf_counter_ns() - t0)
    ts.sort()
    return ts[len(ts) // 2] / 1e3


def cpu_baseline(F, torch, dev, head=None, reps=20, parity_batches=8):
    """The reference math as PyTorch CPU ops (oracle/torch_cpu.py) on the host
    cores, for every configuration, in the same run and on the same kind of
    seeded inputs as the GPU rows: per call with the dequantization (the
    reference's full semantics) and with pre-dequantized bf16-valued fp32
    weights (matmul only, a lower bound); the median of `reps` calls after 3
    warm-ups, GB/s over the GPU rows' algorithmic bytes.  The mixer is timed
    per layer, the LM head's coarse pass on an 8,192-row slice, both scaled
    to the full workload.  Also, with `head`: the fast head's top-512 set and
    argmax against the oracle (numpy, exact coarse sums) on parity_batches
    full-size M = 3 batches."""
    from oracle import torch_cpu as tc
    threads = tc.host_threads()
    torch.set_num_threads(threads)
    g = torch.Generator(device=dev).manual_seed(11)
    cg = torch.Generator().manual_seed(11)
    M, K = 3, 2560
    x = torch.randn((M, K), generator=cg).to(torch.bfloat16)
    rows = {}

    def row(name, nbytes, full, mm, scale=1.0, note=None):
        us_f, us_m = _median_us(full, reps) * scale, _median_us(mm, reps) * scale
        rows[name] = {"us_with_dequant": round(us_f, 1), "us_matmul_only": round(us_m, 1),
                      "GBps_with_dequant": round(nbytes / us_f / 1e3, 3),
                      "GBps_matmul_only": round(nbytes / us_m / 1e3, 3)}
        if note:
            rows[name]["sample"] = note

    def dev_w(n, k):
        return torch.randn((n, k), generator=g, device=dev) * 0.02

    # A: MXFP8 [4096 x 2560]
    q, s = (t.cpu() for t in F.quantize_mx8(dev_w(4096, K)))
    wop = tc.bf16_operand(tc.deq_mx8(q, s))
    row("A_mx8_4096x2560_M3", 4096 * K + 4096 * K // 32 + M * K * 2 + M * 4096 * 2,
        lambda: tc.mx8_linear(x, q, s), lambda: tc.gemv(x, wop))
    # B: 48 router gates [512 x 2560], fp16 scales, fp32 logits
    gates = [tuple(t.cpu() for t in w8_f16(torch, dev_w(512, K))) for _ in range(48)]
    gops = [tc.bf16_operand(tc.deq_w8(qq, ss)) for qq, ss in gates]
    row("B_w8_gates_48_layers_M3", gate_bytes(48, M, 512, K),
        lambda: [tc.w8_linear(x, qq, ss, torch.float32) for qq, ss in gates],
        lambda: [tc.gemv(x, w, torch.float32) for w in gops])
    del gops
    # C: W6 [8192 x 2560] and NVFP4 [16384 x 2560]
    L6, H6, S6 = (t.cpu() for t in F.quantize_w6(dev_w(8192, K)))
    wop = tc.bf16_operand(tc.deq_w6(L6, H6, S6))
    row("C_w6_8192x2560_M3", 8192 * K // 2 + 8192 * K // 4 + 8192 * (K // 32) * 2 + M * K * 2 + M * 8192 * 2,
        lambda: tc.w6_linear(x, L6, H6, S6), lambda: tc.gemv(x, wop))
    P4, S4, gs = F.quantize_nv4(dev_w(16384, K))
    P4, S4 = P4.cpu(), S4.view(torch.uint8).cpu()
    wop = tc.bf16_operand(tc.deq_nv4(P4, S4))
    row("C_nv4_16384x2560_M3", 16384 * K // 2 + 16384 * (K // 16) + 4 + M * K * 2 + M * 16384 * 2,
        lambda: tc.nv4_linear(x, P4, S4, gs), lambda: tc.gemv(x, wop, gs=gs))
    del wop
    # D: one mixer at the synthetic shape (fp32 scales), scaled to 97 layers
    HC, H, ND, LR = 4, 2560, 640, 640
    xd = torch.randn((M, HC * H), generator=cg).to(torch.bfloat16)
    qd, sd = (t.cpu() for t in F.quantize_w8(dev_w(ND, HC * H)))
    qu, su = (t.cpu() for t in F.quantize_w8(dev_w(HC * H, LR)))
    wd, wu = tc.bf16_operand(tc.deq_w8(qd, sd)), tc.bf16_operand(tc.deq_w8(qu, su))

    def mix_mm():
        di = tc.gemv(xd, wd)
        gl = tc.gemv(tc.scaled_silu(di, LR, HC), wu)
        return tc.gate_mean(xd, gl, HC)
    down_b, up_b = mixer_bytes(M, ND, LR, HC, H, 4)
    row("D_hc_mix_one_call_97_layers_M3_f32s", (down_b + up_b) * 97, lambda: tc.mixer(xd, qd, sd, qu, su, LR, HC),
        mix_mm, scale=97.0, note="one mixer timed, times 97")
    # E: the INT2 coarse pass on an 8,192-row slice of the head, scaled to 248,320 rows
    V, NS = 248320, 8192
    P2, S2 = (t.cpu() for t in F.quantize_int2(dev_w(NS, K), group=16))
    wop = tc.bf16_operand(tc.deq_int2(P2, S2))
    row("E_int2_coarse_248320x2560_M3", V * K // 4 + V * (K // 16) * 2 + M * K * 2 + M * V * 2,
        lambda: tc.int2_logits(x, P2, S2, torch.bfloat16), lambda: tc.gemv(x, wop), scale=V / NS,
        note=f"{NS} of {V} rows timed, times {V / NS:.2f}")
    del wop
    res = {"value": rows["B_w8_gates_48_layers_M3"]["GBps_with_dequant"], "unit": "GB/s", "cores": threads,
           "kind": "port",
           "sample": f"48 router gates [512x2560] int8 g64 (fp16 scales) at M=3 as PyTorch CPU ops: dequant, bf16 "
                     f"operand rounding, fp32 matmul, fp32 logits; median of {reps} passes after 3 warm-ups on "
                     f"{threads} host threads",
           "cpu_model": tc.cpu_model(), "torch_version": torch.__version__, "per_config": rows}
    if head is not None:
        res["fast_head_parity"] = head_parity(F, torch, dev, head, parity_batches)
    return res


def head_parity(F, torch, dev, head, batches):
    """The fast head (int2_topk + refine_mx8_, the production calls) on
    `batches` seeded M = 3 batches at full size, against the oracle's fast head
    (exact coarse sums rounded to fp32 then bf16, the total-order top-512, the
    rescore's fma order): the share of rows whose top-512 set is identical,
    and of rows whose argmax is; and the argmax agreement over every vector of
    the GPU leg's 1,000-vector argmax row (head[4]: the vectors and the fast
    head's argmaxes), against the oracle's fast head on the same vectors."""
    import numpy as np
    from oracle import formats as fm
    from oracle import head as oh
    q, s, P, S, (x_all, fast_am) = head
    V, K, C, M = P.shape[0], P.shape[1] * 4, 512, 3
    xs, sel, outs = [], [], []
    for b in range(batches):
        gx = torch.Generator(device=dev).manual_seed(5000 + b)
        x = torch.randn((M, K), generator=gx, device=dev).to(torch.bfloat16)
        co, ix = F.int2_topk(x, P, S, V, C, sorted=False)
        out = F.refine_mx8_(co, x, ix, q, s)
        xs.append(x.view(torch.int16).cpu().numpy().view(np.uint16))
        sel.append(ix.cpu().numpy())
        outs.append(out.view(torch.int16).cpu().numpy().view(np.uint16))
    xb, sel, outs = np.concatenate(xs), np.concatenate(sel), np.concatenate(outs)
    Pn, Sn, qn, sn = P.cpu().numpy(), S.cpu().numpy(), q.view(torch.uint8).cpu().numpy(), s.cpu().numpy()
    import _fp4x
    o_coarse, o_idx, o_out = oh.fast_head(xb, Pn, Sn, 16, qn, sn, C, _fp4x.layout(_fp4x.FMT_MX8, K)[0])
    same_set = float(np.mean([set(a) == set(b) for a, b in zip(sel.tolist(), o_idx.tolist())]))
    am = np.argmax(fm.bf16_to_f32(outs), -1)
    am_o = np.argmax(fm.bf16_to_f32(o_out), -1)
    res = {"rows": int(xb.shape[0]), "top512_set_identity_vs_oracle": round(same_set, 4),
           "argmax_agreement_vs_oracle": round(float(np.mean(am == am_o)), 4)}
    # the argmax of every one of the 1,000 vectors behind the fast head's argmax_agreement row, against the
    # oracle's fast head on the same vectors
    t0 = time.perf_counter()
    am_all = oh.fast_head_argmax(x_all.numpy().view(np.uint16), Pn, Sn, 16, qn, sn, C,
                                 _fp4x.layout(_fp4x.FMT_MX8, K)[0])
    res["argmax_agreement_vs_oracle_all_vectors"] = round(float(np.mean(am_all == fast_am.numpy())), 4)
    res["all_vectors"] = int(am_all.size)
    res["all_vectors_cpu_s"] = round(time.perf_counter() - t0, 1)
    return res


# ------------------------------------------------------------------ main
def main():
    args = parse()
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy, args.steps)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: only --gpus 1 is supported: these kernels are measured on one GPU and no "
              "multi-GPU figure is produced", file=sys.stderr)
        sys.exit(2)
    import torch
    import fp4x_kernels as F
    dev = torch.device("cuda:0")
    torch.manual_seed(0)

    # headline: 48 router gates in one layer-batched launch, rotated copies
    L, M, n, k = 48, 3, 512, 2560
    q, s = gate_weights(F, torch, dev, L, n, k)
    step_bytes = gate_bytes(L, M, n, k)
    ncp = copies_for(L * (n * k + n * (k // 64) * 2))
    qs = [(q.clone(), s.clone()) for _ in range(ncp - 1)] + [(q, s)]
    x3 = torch.randn((L, M, k), device=dev).to(torch.bfloat16)
    out3 = [torch.empty((L, M, n), dtype=torch.float32, device=dev) for _ in range(ncp)]
    lib = F._L.lib()

    def step(i):
        qq, ss = qs[i % ncp]
        F._L.check(lib.fp4x_w8_linear_layers(F._ptr(x3), k, M * k, F._ptr(qq), n * k, F._ptr(ss), F._L.DT_F16,
                                             n * (k // 64), F._ptr(out3[i % ncp]), F._L.DT_F32, M * n, L, M, n, k,
                                             1, None, None, F._L.stream_of(x3)), "gates")

    # sanity of the timed path against the per-layer entry point (a different
    # kernel, the same fp32 sum up to summation order)
    y = F.w8_linear_layers(x3, q, s, torch.float32)
    y1 = F.w8_linear(x3[7], q[7], s[7], (16, 512, 1, 4), torch.float32)
    assert torch.allclose(y[7], y1, rtol=2e-3, atol=1e-2)

    # K steps run as replays of one graph holding G consecutive steps (every
    # weight copy in turn, so launches follow each other without replay gaps),
    # plus one graph for the K mod G remainder: exactly K launches are timed.
    G = ncp * 8
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())

    def capture(nsteps):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=cs):
            for i in range(nsteps):
                step(i)
        return gr

    with torch.cuda.stream(cs):
        step(0)
        torch.cuda.synchronize()
        g_full = capture(G)
        rem = args.steps % G
        g_rem = capture(rem) if rem else None
        for _ in range(args.warmup // G):
            g_full.replay()
        for i in range(args.warmup % G):
            step(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(cs)
        for _ in range(args.steps // G):
            g_full.replay()
        if g_rem is not None:
            g_rem.replay()
        e1.record(cs)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / args.steps
    value = step_bytes / (ms_step * 1e-3) / 1e9

    kernels = {}
    kernels["B_w8_gates_48_layers_M3"] = entry(ms_step * 1e3, step_bytes)
    sel = set("ABCDEFGHI") if args.kernels == "all" else set() if args.kernels == "none" else set(args.kernels.split(","))
    def done(what):
        print(f"[bench] {what} done", file=sys.stderr, flush=True)

    done("headline")
    if "B" in sel:
        bench_gates_single(F, torch, dev, kernels, q, s)
        done("B")
    del qs, out3, g_full, g_rem
    torch.cuda.empty_cache()
    if sel & {"A", "C"}:
        bench_dense(F, torch, dev, kernels)
        done("A, C")
    if "D" in sel:
        bench_hc(F, torch, dev, kernels)
        torch.cuda.empty_cache()
        done("D")
    head = None
    if "E" in sel:
        head = bench_head(F, torch, dev, kernels)
        torch.cuda.empty_cache()
        done("E")
    if "F" in sel:
        bench_draft(F, torch, dev, kernels)
        torch.cuda.empty_cache()
        done("F")
    if "G" in sel:
        bench_prep(F, torch, dev, kernels)
        torch.cuda.empty_cache()
        done("G")
    if "H" in sel:
        bench_mtp(F, torch, dev, kernels)
        torch.cuda.empty_cache()
        done("H")
    if "I" in sel:
        bench_shapes(F, torch, dev, kernels)
        torch.cuda.empty_cache()
        done("I")

    ceil = {}
    if not args.no_ceiling:
        ceil = bench_read_ceiling(F, torch, dev, ceiling_sizes(kernels))
        attach_ceilings(kernels, ceil)
        done("read ceilings")
    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic_gates48_M3.json")
    if os.path.exists(tf):
        traffic = json.load(open(tf)).get("hbm_bytes_per_launch")
    line = {
        "metric": "per-kernel µs + achieved HBM GB/s (% of MI355X peak) at M=1/3/16",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights quantized on device, N(0,1) bf16 activations)",
        "config": {"workload": "int8 g64 router gates: 48 layers x [512 x 2560], M=3, fp16 scales, fp32 logits, "
                               "one layer-batched launch per step",
                   "layers": L, "M": M, "N": n, "K": k, "weight_copies_rotated": ncp,
                   "bytes_per_step": step_bytes, "wall_s": round(wall, 3)},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / PEAK_GBS, 4), "traffic": traffic},
        "kernels": kernels,
        "read_ceiling": {f"{nb / 1e6:.2f}MB": {"us": round(c[0], 3), "GBps": round(nb / c[0] / 1e3, 1),
                                                "shape": c[1]} for nb, c in sorted(ceil.items())},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(F, torch, dev, head)
        done("cpu baseline")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
