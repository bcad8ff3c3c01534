"""The PyTorch CPU restatement (oracle/torch_cpu.py, the benchmark's CPU
baseline) against the numpy oracle: every dequantized operand bit for bit,
GEMV sums within the fp32 summation-order bound, the mixer epilogues and the
fast head's selection and rescore."""
import numpy as np
import torch

from oracle import formats as fm
from oracle import gemv as og
from oracle import head as oh
from oracle import hc as ohc
from oracle import ordered
from oracle import quant as oq
from oracle import torch_cpu as tc


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def _bf16(a):
    return _t(fm.bf16_bits(a).view(np.int16)).view(torch.bfloat16)


def _setup(seed=0, n=96, k=256, m=3):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = fm.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    return rng, w, x


def test_dequant_operands_bit_exact():
    _, w, _ = _setup()
    q, s = oq.quantize_mx8(w)
    assert np.array_equal(tc.deq_mx8(_t(q), _t(s)).numpy(), oq.mx8_dequant(q, s))
    q8, s8 = oq.quantize_w8(w)
    assert np.array_equal(tc.deq_w8(_t(q8), _t(s8)).numpy(), oq.dequant_w8(q8, s8))
    L, H, S = oq.quantize_w6(w)
    assert np.array_equal(tc.deq_w6(_t(L), _t(H), _t(S)).numpy(), oq.dequant_w6(L, H, S))
    P, S4, gs = oq.quantize_nv4(w)
    assert np.array_equal(tc.deq_nv4(_t(P), _t(S4)).numpy(), oq.dequant_nv4_operand(P, S4))
    P2, S2 = oq.quantize_int2(w)
    assert np.array_equal(tc.deq_int2(_t(P2), _t(S2)).numpy(), oq.dequant_int2(P2, S2))


def _within(got, x, w_op, gs=1.0):
    exact = ordered.exact_sum(x, w_op) * gs
    bound = (w_op.shape[1] + 2) * 2.0 ** -23 * ordered.exact_sum(np.abs(x), np.abs(w_op)) * abs(gs)
    bound = bound + np.abs(exact) * 2.0 ** -8                      # bf16 output rounding
    return np.all(np.abs(np.asarray(got, np.float64) - exact) <= bound)


def test_gemvs_within_summation_bound():
    _, w, x = _setup(1)
    xt = _bf16(x)
    q, s = oq.quantize_mx8(w)
    assert _within(tc.mx8_linear(xt, _t(q), _t(s)).float().numpy(), x, og.operand("mx8", q, s))
    q8, s8 = oq.quantize_w8(w)
    assert _within(tc.w8_linear(xt, _t(q8), _t(s8)).float().numpy(), x, og.operand("w8", q8, s8))
    L, H, S = oq.quantize_w6(w)
    assert _within(tc.w6_linear(xt, _t(L), _t(H), _t(S)).float().numpy(), x, og.operand("w6", L, H, S))
    P, S4, gs = oq.quantize_nv4(w)
    assert _within(tc.nv4_linear(xt, _t(P), _t(S4), gs).float().numpy(), x, og.operand("nv4", P, S4), gs)
    P2, S2 = oq.quantize_int2(w)
    assert _within(tc.int2_logits(xt, _t(P2), _t(S2)).numpy(), x, og.operand("int2", P2, S2))


def test_mixer_epilogues_equal_oracle():
    rng = np.random.default_rng(2)
    d = fm.round_bf16((rng.standard_normal((3, 640)) * 3).astype(np.float32))
    bot = tc.scaled_silu(_bf16(d), 640, 4)
    # torch's CPU sigmoid may differ from the correctly rounded one in the last
    # fp32 bit; after the bf16 rounding the two agree on all but rare inputs
    ref = ohc.scaled_silu(d, 4)
    agree = (bot.view(torch.int16).numpy().view(np.uint16) == fm.bf16_bits(ref)).mean()
    assert agree > 0.999
    nrm = fm.round_bf16(rng.standard_normal((3, 4 * 256)).astype(np.float32))
    g = fm.round_bf16((rng.standard_normal((3, 4 * 256)) * 2).astype(np.float32))
    out = tc.gate_mean(_bf16(nrm), _bf16(g), 4)
    ref = ohc.gate_mean(nrm, g, 4)
    assert (out.view(torch.int16).numpy().view(np.uint16) == fm.bf16_bits(ref)).mean() > 0.999


def test_fast_head_selection_and_rescore():
    rng = np.random.default_rng(3)
    V, K, C = 2048, 256, 64
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    w[rng.choice(V, 8, replace=False)] *= 4
    q, s = oq.quantize_mx8(w)
    P, S = oq.quantize_int2(oq.mx8_dequant(q, s))
    x = fm.round_bf16(rng.standard_normal((2, K)).astype(np.float32))
    out, idx = tc.fast_head(_bf16(x), _t(P), _t(S), _t(q), _t(s), C)
    coarse = tc.int2_logits(_bf16(x), _t(P), _t(S), torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    sel = idx.numpy()
    want = oh.topk_total_order(coarse, C)
    key = oh.order_keys(coarse)
    for r in range(2):
        # torch.topk leaves the order among equal values open: the same set
        # up to elements tied with the C-th largest value
        kth = key[r, want[r, -1]]
        assert np.all(key[r, sel[r]] >= kth)
        assert set(np.flatnonzero(key[r] > kth)) <= set(sel[r].tolist())
    got = np.take_along_axis(out.view(torch.int16).numpy().view(np.uint16), sel, 1)
    exact = oh.mx8_rows(fm.bf16_bits(x), q, s, sel, 4)
    f = fm.bf16_to_f32
    assert np.all(np.abs(f(got) - f(fm.bf16_bits(exact))) <= np.abs(f(fm.bf16_bits(exact))) * 2.0 ** -7)
