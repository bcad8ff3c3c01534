"""Entry points with state kept across calls (split-K tickets, the single-launch
mixer's count and flags, the top-k workspace) replayed from HIP graphs, as the
plugin runs them under vLLM's decode-graph capture: every replay, with eager
work and synchronizations between replays, equals the eager results bit for
bit, and the scratch is re-armed after each replay."""
import numpy as np
import pytest
import torch

from gpu_helpers import act, bf16_dev, path_switch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def F():
    import fp4x_kernels
    return fp4x_kernels


def replay_and_check(fn, expected, eager_between):
    """Capture fn() once, replay it three times; after each replay check every
    output against the eager results, then run eager work before the next."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                                       # warm-up outside the capture (allocations, workspaces)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            outs = fn()
    torch.cuda.synchronize()
    for r in range(3):
        for o in outs:
            o.fill_(0)                             # a stale value cannot pass for a replayed one
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, expected)):
            assert torch.equal(o, e), f"replay {r} output {i}"
        eager_between()
        torch.cuda.synchronize()


def test_graph_mixer_one_launch(gpu, F):
    HC, H, LR, ND = 4, 2560, 320, 336
    gen = torch.Generator(device=gpu).manual_seed(5)
    fx = F.HCFused(gpu)
    layers = []
    for _ in range(4):
        qd, sd = F.quantize_w8(torch.randn((ND, HC * H), generator=gen, device=gpu) * 0.02)
        qu, su = F.quantize_w8(torch.randn((HC * H, LR), generator=gen, device=gpu) * 0.02)
        qi, si = F.HCFused.interleave_up(qu, su, HC, 8)
        layers.append((qd, sd, qi, si))
    x = bf16_dev(act(np.random.default_rng(5), 3, HC * H)[0])
    cfg = (32, 256, 8, 4)

    def run():
        outs = []
        for qd, sd, qi, si in layers:
            outs += list(fx.mix(x, qd, sd, LR, HC, qi, si, x, cfg))
        return outs

    expected = []
    for qd, sd, qi, si in layers:                 # the two-call reference, eagerly
        di, bot = fx.down(x, qd, sd, LR, HC, cfg)
        expected += [di, bot, F.HCFused.up(bot, qi, si, x, HC, (8, 64, 4))]
    torch.cuda.synchronize()

    def eager():
        fx.mix(x, *layers[0][:2], LR, HC, *layers[0][2:], x, cfg)
        assert int(fx.tickets[:fx._status_at].abs().sum()) == 0

    replay_and_check(run, expected, eager)
    assert int(fx.tickets[:fx._status_at].abs().sum()) == 0


@pytest.mark.parametrize("rows", ["1", "0"])
def test_graph_splitk_and_gates(gpu, F, rows, monkeypatch):
    """The mixer-shaped W8 GEMV (640 x 10240, 4 K slices) and the 48-layer
    gates under replay: with the few-rows kernels (default) and with the
    split-K tile kernel and its tickets (FP4X_ROWS=0)."""
    gen = torch.Generator(device=gpu).manual_seed(6)
    q, s = F.quantize_w8(torch.randn((640, 10240), generator=gen, device=gpu) * 0.02)
    x = torch.randn((3, 10240), generator=gen, device=gpu).to(torch.bfloat16)
    qg, sg = F.quantize_w8(torch.randn((48 * 512, 2560), generator=gen, device=gpu) * 0.02)
    qg, sg = qg.view(48, 512, 2560), sg.view(48, 512, 40).half()
    xg = torch.randn((48, 3, 2560), generator=gen, device=gpu).to(torch.bfloat16)

    def run():
        return [F.w8_linear(x, q, s, (32, 256, 4, 4), torch.float32),
                F.w8_linear_layers(xg, qg, sg, torch.float32)]

    with path_switch(monkeypatch, "FP4X_ROWS", rows):
        expected = run()
        torch.cuda.synchronize()
        replay_and_check(run, [e.clone() for e in expected],
                         lambda: F.w8_linear(x[:1], q, s, (32, 256, 4, 4), torch.float32))


def test_graph_int2_topk(gpu, F):
    V, K, C = 248320, 2560, 512
    gen = torch.Generator(device=gpu).manual_seed(7)
    w = torch.randn((V, K), generator=gen, device=gpu) * 0.02
    P, S = F.quantize_int2(w, group=16)
    del w
    x = torch.randn((3, K), generator=gen, device=gpu).to(torch.bfloat16)

    def run():
        coarse, idx = F.int2_topk(x, P, S, V, C)
        return [coarse, idx]

    expected = [e.clone() for e in run()]
    torch.cuda.synchronize()
    replay_and_check(run, expected, lambda: F.topk_rows(expected[0], C))


def test_graph_draft_head(gpu, F):
    """The draft head's INT2 coarse + top-64 + NVFP4 rescore + scatter
    (fp4patch._draft_logits), with a device temperature scalar, replayed."""
    import fp4patch
    V, K, NS, DC = 60000, 2560, 20000, 64
    gen = torch.Generator(device=gpu).manual_seed(8)
    P, S, gs = F.quantize_nv4(torch.randn((V, K), generator=gen, device=gpu) * 0.02)
    ids = torch.sort(torch.randperm(V, generator=gen, device=gpu)[:NS]).values
    st = fp4patch._draft_prepare(F, P, S, gs, ids, DC)
    x = torch.randn((3, K), generator=gen, device=gpu).to(torch.bfloat16)
    inv_t = torch.full((1,), 1.25, device=gpu)

    def run():
        return [fp4patch._draft_logits(F, x, st, V, DC, inv_t=inv_t)]

    expected = [e.clone() for e in run()]
    torch.cuda.synchronize()
    replay_and_check(run, expected, lambda: F.refine_nv4(x, torch.zeros((3, DC), dtype=torch.int64, device=gpu),
                                                         st["w"], st["s"], st["gs"]))


def test_graph_topk_workspace_grows_after_capture(gpu, F):
    """A graph captured on a small top-k workspace keeps replaying correctly
    after an eager call grows the workspace (the old buffer stays alive), and
    growing it during a capture raises instead of handing the graph a buffer
    sized for one call."""
    gen = torch.Generator(device=gpu).manual_seed(9)
    F._TOPK_WS.clear()
    small = torch.randn((2, 5000), generator=gen, device=gpu).to(torch.bfloat16)
    big = torch.randn((16, 300000), generator=gen, device=gpu).to(torch.bfloat16)

    def run():
        return [F.topk_rows(small, 64)]

    expected = [e.clone() for e in run()]
    torch.cuda.synchronize()
    replay_and_check(run, expected, lambda: F.topk_rows(big, 512))   # the eager call grows the workspace
    F._TOPK_WS.clear()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="workspace too small"):
            with torch.cuda.graph(g, stream=s):
                F.topk_rows(big, 512)
    torch.cuda.synchronize()
