"""Benchmark of the fp4x decode GEMVs on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--kernels all|none|A,B,...]

Headline (one JSON line): the int8 g64 router-gate GEMV of a decode step —
48 independent [512 x 2560] gates at M = 3 (1 target + 2 draft rows), one
fp16 scale per 64 K values, fp32 logits — as one layer-batched launch.  A step is one such launch
over one batch of synthetic input; `value` is algorithmic bytes (weights +
scales + activations + logits) per second with all inputs resident in HBM.
Weights rotate through copies totalling > 512 MB so every launch streams from
HBM rather than the 256 MB MALL.

`kernels` adds per-kernel µs and GB/s for every configuration (MXFP8 4096 x
2560, W6 8192 x 2560, NVFP4 16384 x 2560 at M = 1/3/16, the 97-layer fused
mixer, the 248,320-row fast LM head and the exact MXFP8 head it replaces, the
65k-token draft head), timed as
HIP-graph replays, and the load-time weight preparation (group G, eager).
`cpu_baseline` times the oracle (numpy) on the host cores for a bounded
sample of the headline workload.
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
    ap.add_argument("--kernels", default="all", help="all | none | comma list of A,B,C,D,E,F,G")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
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


def bench_gates_single(F, torch, dev, out, q, s):
    M, n, k = 3, 512, 2560
    x = torch.randn((M, k), device=dev).to(torch.bfloat16)
    calls = [lambda i=i: F.w8_linear(x, q[i], s[i], (16, 512, 1, 4), torch.float32) for i in range(q.shape[0])]
    us = graph_time(calls)
    out["B_w8_gate_single_layer_M3"] = entry(us, gate_bytes(1, M, n, k))


def bench_hc(F, torch, dev, out, layers=97):
    HC, H, LR, ND, KS, M = 4, 2560, 640, 640, 16, 3
    g = torch.Generator(device=dev).manual_seed(1)
    fx = F.HCFused(dev, n_down=ND, max_ksplit=KS)
    mix = []
    for _ in range(layers):
        qd, sd = w8_f16(torch, torch.randn((ND, HC * H), generator=g, device=dev) * 0.02)
        qu, su = w8_f16(torch, torch.randn((HC * H, LR), generator=g, device=dev) * 0.02)
        qi, si = F.HCFused.interleave_up(qu, su, HC, 8)
        mix.append((qd, sd, qi, si))
    x = torch.randn((M, HC * H), generator=g, device=dev).to(torch.bfloat16)
    down_b = ND * HC * H + ND * (HC * H // 64) * 2 + M * HC * H * 2 + M * ND * 2 + M * LR * 2
    up_b = HC * H * LR + HC * H * (LR // 64) * 2 + M * LR * 2 + M * HC * H * 2 + M * H * 2
    bots = [fx.down(x, qd, sd, LR, HC, (32, 256, KS, 4))[1] for qd, sd, _, _ in mix]
    us_down = graph_time([lambda m=m: fx.down(x, m[0], m[1], LR, HC, (32, 256, KS, 4)) for m in mix], replays=5)
    us_up = graph_time([lambda m=m, b=b: F.HCFused.up(b, m[2], m[3], x, HC, (8, 64, 4)) for m, b in zip(mix, bots)],
                       replays=5)

    def both(m):
        _, bot = fx.down(x, m[0], m[1], LR, HC, (32, 256, KS, 4))
        F.HCFused.up(bot, m[2], m[3], x, HC, (8, 64, 4))
    us_pair = graph_time([lambda m=m: both(m) for m in mix], replays=5)
    # the whole mixer as one call (one launch per mixer at this shape)
    us_mix = graph_time([lambda m=m: fx.mix(x, m[0], m[1], LR, HC, m[2], m[3], x, (32, 256, KS, 4)) for m in mix],
                        replays=5)
    out["D_hc_down_640x10240_M3"] = entry(us_down, down_b)
    out["D_hc_up_10240x640_M3"] = entry(us_up, up_b)
    out["D_hc_mixer_97_layers_M3"] = entry(us_pair * layers, (down_b + up_b) * layers)
    out["D_hc_mixer_97_layers_M3"]["us_per_mixer"] = round(us_pair, 3)
    out["D_hc_mix_one_call_97_layers_M3"] = entry(us_mix * layers, (down_b + up_b) * layers)
    out["D_hc_mix_one_call_97_layers_M3"]["us_per_mixer"] = round(us_mix, 3)


def bench_head(F, torch, dev, out, vectors=1000):
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
    coarse = F.int2_logits(x, P, S, V, out_dtype=torch.bfloat16)
    us = graph_time([lambda: F.topk_rows(coarse, C)] * 4, 10)
    out["E_topk512_M3"] = entry(us, M * V * 2 + M * C * 8)
    # the coarse pass and the top-C in one call (slice maxima from the coarse kernel)
    us = graph_time([lambda c=c: F.int2_topk(x, c[0], c[1], V, C) for c in copies], 10)
    out["E_int2_coarse_plus_topk512_M3"] = entry(us, int2_b + M * C * 8)
    idx = F.topk_rows(coarse, C)
    us = graph_time([lambda: F.refine_mx8_(coarse, x, idx, q, s)] * 4, 10)
    out["E_refine_mx8_3x512_M3"] = entry(us, M * C * (K + K // 32 + 8) + M * K * 2 + M * C * 2)

    def head(xx, c):
        co, ix = F.int2_topk(xx, c[0], c[1], V, C)
        F.refine_mx8_(co, xx, ix, q, s)
    us = graph_time([lambda c=c: head(x, c) for c in copies], 10)
    out["E_fast_head_total_M3"] = {"us": round(us, 3)}
    # the exact head the fast path replaces: the MXFP8 GEMV over all 248,320 rows
    # (655 MB, above the 256 MB MALL, so one copy streams from HBM)
    us = graph_time([lambda: F.mx8_linear(x, q, s, (32, 512, 1, 4))] * 2, 10)
    out["E_exact_head_mx8_248320x2560_M3"] = entry(us, V * K + V * K // 32 + M * K * 2 + M * V * 2)
    # argmax agreement against the exact-weight MXFP8 GEMV over seeded vectors
    agree, n = 0, 0
    for b0 in range(1000, 1000 + vectors, M):
        rng = torch.Generator(device=dev).manual_seed(b0)
        xs = torch.randn((M, K), generator=rng, device=dev).to(torch.bfloat16)
        co, ix = F.int2_topk(xs, P, S, V, C)
        fast = F.refine_mx8_(co, xs, ix, q, s)
        full = F.mx8_linear(xs, q, s, (32, 512, 1, 4))
        m = min(M, 1000 + vectors - b0)
        agree += int((fast[:m].argmax(-1) == full[:m].argmax(-1)).sum())
        n += m
    out["E_fast_head_total_M3"]["argmax_agreement"] = round(agree / n, 4)
    out["E_fast_head_total_M3"]["vectors"] = n


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
    cand = F.int2_topk(x, *st["c"], NS, DC)[1]
    us = graph_time([lambda: F.refine_nv4(x, cand, st["w"], st["s"], st["gs"])] * 4, 10)
    out["F_refine_nv4_3x64_M3"] = entry(us, M * DC * (K // 2 + K // 16 + 8) + M * K * 2 + M * DC * 4)
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


def cpu_baseline(seconds):
    """The oracle's dequantize-then-matmul router gates (numpy, all host
    cores) on a bounded sample: whole 48-layer passes at M = 3."""
    import numpy as np
    from oracle import gemv as og, quant as oq, formats as fm
    cores = len(os.sched_getaffinity(0))
    rng = np.random.default_rng(0)
    layers = [oq.quantize_w8((rng.standard_normal((512, 2560)) * 0.02).astype(np.float32)) for _ in range(48)]
    layers = [(q, s.astype(np.float16).astype(np.float32)) for q, s in layers]     # fp16 scale values
    x = fm.round_bf16(rng.standard_normal((3, 2560)).astype(np.float32))
    passes, t0 = 0, time.perf_counter()
    while True:
        for q, s in layers:
            og.w8_linear(x, q, s, "f32")
        passes += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = (time.perf_counter() - t0) / passes
    nbytes = gate_bytes(48, 3, 512, 2560)
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "ms_per_step": round(dt * 1e3, 2),
            "sample": f"{passes} passes of 48 router gates [512x2560] int8 g64 at M=3 (numpy dequant, bf16 "
                      f"operand rounding, fp32 matmul; {cores} host threads)"}


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
    sel = set("ABCDEFG") if args.kernels == "all" else set() if args.kernels == "none" else set(args.kernels.split(","))
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
    if "E" in sel:
        bench_head(F, torch, dev, kernels)
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
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
