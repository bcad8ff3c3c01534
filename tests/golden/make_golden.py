"""Writes tests/golden/quant_golden.npz: input/output vectors of the
reference plugin's pure-torch weight-preparation functions
(x/fp4x_kernels.py: quantize_w8 :138-144, quantize_w6 :179-202,
mx8_dequant :261-267, quantize_nv4 :277-300, quantize_int2 :330-351,
dequant_int2 :353-357, dequant_nv4 :420-426, HCFused.interleave_up :512-517).

Run once in the build container, where the reference tree is mounted:
    python tests/golden/make_golden.py /root/reference/x
It imports only that module (torch + triton at import; no kernel runs) on CPU
tensors.  The fixture holds data only; GPU runs never read the reference.
"""
import importlib.util
import os
import sys

import numpy as np
import torch


def load_reference(xdir):
    spec = importlib.util.spec_from_file_location("ref_fp4x_kernels", os.path.join(xdir, "fp4x_kernels.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def ties_w8():
    """Rows whose g64 scale is a power of two, with values at .5 steps."""
    s = 2.0 ** -6
    row = np.zeros(128, np.float32)
    row[0] = 127 * s
    row[1:9] = np.array([2.5, -3.5, 0.5, -0.5, 1.5, 126.5, -126.5, 63.5]) * s
    row[64] = -127 * s
    row[65:70] = np.array([4.5, -4.5, 5.5, 0.49999997, -1.5]) * s
    return row


def ties_w6():
    s = 2.0 ** -8
    row = np.zeros(128, np.float32)
    row[0] = 31 * s
    row[1:8] = np.array([2.5, -3.5, 30.5, -30.5, 0.5, -0.5, 7.5]) * s
    row[32] = -31 * s
    row[33:36] = np.array([-29.5, 1.5, -2.5]) * s
    return row


def main(xdir):
    F = load_reference(xdir)
    g = torch.Generator().manual_seed(1234)
    out = {}

    w = (torch.randn(8, 128, generator=g) * 0.02)
    w[7] = torch.from_numpy(ties_w8())
    q, s = F.quantize_w8(w)
    out.update(w8_w=w.numpy(), w8_q=q.numpy(), w8_s=s.numpy())

    w = (torch.randn(8, 128, generator=g) * 0.02)
    w[7] = torch.from_numpy(ties_w6())
    L, H, S = F.quantize_w6(w)
    out.update(w6_w=w.numpy(), w6_L=L.numpy(), w6_H=H.numpy(), w6_S=S.numpy())
    L, H, S = F.quantize_w6(w, qmax=15, clip_search=3)
    out.update(w6c_L=L.numpy(), w6c_H=H.numpy(), w6c_S=S.numpy())

    codes = (torch.randn(8, 64, generator=g) * 0.5).to(torch.float8_e4m3fn)
    exps = torch.randint(118, 126, (8, 2), generator=g, dtype=torch.uint8)
    out.update(mx8_w=codes.view(torch.uint8).numpy(), mx8_s=exps.numpy(),
               mx8_deq=F.mx8_dequant(codes, exps).numpy())

    w = (torch.randn(8, 64, generator=g) * 0.02)
    w[3, :16] = 0.0
    P, S, gs = F.quantize_nv4(w)
    out.update(nv4_w=w.numpy(), nv4_P=P.numpy(), nv4_S=S.view(torch.uint8).numpy(), nv4_gs=np.float64(gs),
               nv4_deq=F.dequant_nv4(P, S, gs).numpy())

    w = (torch.randn(8, 128, generator=g) * 0.02)
    w[5, :32] = 0.0
    for grp in (16, 32):
        P, S = F.quantize_int2(w, group=grp)
        out.update(**{f"int2g{grp}_P": P.numpy(), f"int2g{grp}_S": S.numpy(),
                      f"int2g{grp}_deq": F.dequant_int2(P, S).numpy()})
    P, S, R = F.quantize_int2(w, scale_fmt="e4m3", group=16)
    out.update(int2e_P=P.numpy(), int2e_S=S.view(torch.uint8).numpy(), int2e_R=R.numpy())
    out.update(int2_w=w.numpy())

    q = torch.arange(32 * 4, dtype=torch.int32).view(32, 4).to(torch.int8)
    s = torch.arange(32 * 1, dtype=torch.float32).view(32, 1)
    qi, si = F.HCFused.interleave_up(q, s, 4, 2)
    out.update(il_q=q.numpy(), il_qi=qi.numpy(), il_si=si.numpy())

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quant_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/x")
