"""Shared helpers of the GPU parity tests (numpy <-> device tensors)."""
import contextlib

import numpy as np
import torch

from oracle import formats as fm


def dev(a, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def bf16_dev(x, device="cuda"):
    """fp32 array -> bf16 device tensor (round to nearest even)."""
    return dev(fm.bf16_bits(x).view(np.int16), device).view(torch.bfloat16)


def bf16_bits(t):
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def to_f32(t):
    if t.dtype == torch.bfloat16:
        return fm.bf16_to_f32(bf16_bits(t))
    return t.detach().float().cpu().numpy()


def act(rng, M, K):
    """bf16-valued activations ~ N(0, 1) as fp32, and the bits."""
    x = fm.round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    return x, fm.bf16_bits(x)


def assert_tol(got, ref, rel=2e-3, abs_=1e-2, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    bad = np.abs(got - ref) > abs_ + rel * np.abs(ref)
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside |d| <= {abs_} + {rel}|ref|; "
                           f"max |d| {np.abs(got - ref).max():.3g}")


@contextlib.contextmanager
def path_switch(monkeypatch, name, value="0"):
    """Set one of the library's FP4X_* path switches for the block (the
    library reads them once, so each change is followed by a reload)."""
    import _fp4x
    monkeypatch.setenv(name, value)
    _fp4x.reload_env()
    try:
        yield
    finally:
        monkeypatch.delenv(name, raising=False)
        _fp4x.reload_env()
