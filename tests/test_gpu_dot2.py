"""Measures the rounding of v_dot2_f32_bf16 against the oracle's models.

The instruction is not a correctly rounded three-term sum: on random
operands it agrees with RN(a0*b0 + a1*b1 + c) for about 88% of inputs and
with chained IEEE fma for about 84%.  No GEMV accumulates with it (the dense
cores use MFMA, the rescore uses IEEE fma); the test bounds its error by
2^-23 * (|a0 b0| + |a1 b1| + |c|) and records the agreement rates."""
import numpy as np
import pytest
import torch

from oracle import ordered

from gpu_helpers import dev


def bits_pair(a0, a1):
    from oracle import formats as fm
    lo = int(fm.bf16_bits(np.array([a0], np.float32))[0])
    hi = int(fm.bf16_bits(np.array([a1], np.float32))[0])
    return lo | (hi << 16)


def operands(rng, n):
    """Random bf16 pairs with spread exponents, and accumulators near the
    products' magnitudes so the roundings differ between candidate models."""
    def bf(shape, lo, hi):
        mant = rng.integers(0x80, 0x100, shape).astype(np.uint32)     # 8 significant bits
        exp = rng.integers(lo, hi, shape).astype(np.uint32)
        sign = rng.integers(0, 2, shape).astype(np.uint32)
        return ((sign << 15) | (exp << 7) | (mant & 0x7F)).astype(np.uint32)
    a = bf(n, 110, 140) | (bf(n, 110, 140) << 16)
    b = bf(n, 110, 140) | (bf(n, 110, 140) << 16)
    c = (rng.standard_normal(n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    return a, b, c


@pytest.mark.gpu
def test_dot2_rounding_model(gpu):
    import _fp4x
    rng = np.random.default_rng(11)
    a, b, c = operands(rng, 1 << 20)
    # crafted: c = 1, products 2^-24 each (sequential rounding loses both, a fused sum keeps them)
    crafted = [(bits_pair(2.0 ** -12, 2.0 ** -12), bits_pair(2.0 ** -12, 2.0 ** -12), 1.0),
               (bits_pair(1.0, 2.0 ** -24), bits_pair(1.0, 1.0078125), 2.0 ** -25),
               (bits_pair(3.0, -3.0), bits_pair(2.0 ** 20, 2.0 ** 20), 1.0),
               (bits_pair(1.0, 1.0), bits_pair(2.0 ** -25, 2.0 ** -25), 1.0)]
    a = np.concatenate([np.array([t[0] for t in crafted], np.uint32), a])
    b = np.concatenate([np.array([t[1] for t in crafted], np.uint32), b])
    c = np.concatenate([np.array([t[2] for t in crafted], np.float32), c])
    out = torch.empty(len(a), dtype=torch.float32, device=gpu)
    A, B, Cc = dev(a.view(np.int32)), dev(b.view(np.int32)), dev(c)
    _fp4x.check(_fp4x.lib().fp4x_dot2_bf16(_fp4x.ptr(A), _fp4x.ptr(B), _fp4x.ptr(Cc), _fp4x.ptr(out), len(a),
                                           _fp4x.stream_of(out)), "dot2")
    got = out.cpu().numpy()
    report = {}
    for mode in range(4):
        want = ordered.dot2(a, b, c, mode)
        report[mode] = float(np.mean(got.view(np.uint32) == want.view(np.uint32)))
    print(f"dot2 agreement per model: {report}; crafted gpu={got[:4].tolist()}")
    rn = ordered.dot2(a, b, c, 0).astype(np.float64)

    def halves(v):
        lo = (v & 0xFFFF).astype(np.uint32) << 16
        hi = v & 0xFFFF0000
        return lo.view(np.float32).astype(np.float64), hi.view(np.float32).astype(np.float64)
    a0, a1 = halves(a)
    b0, b1 = halves(b)
    l1 = np.abs(a0 * b0) + np.abs(a1 * b1) + np.abs(c.astype(np.float64))
    err = np.abs(got.astype(np.float64) - rn)
    assert np.all(err <= 2.0 ** -23 * l1), float((err / (2.0 ** -23 * l1)).max())
    assert report[0] >= 0.8
