"""PyTorch CPU restatement of the reference's dequantize-then-matmul math
(oracle; test infrastructure only).

The benchmark's CPU baseline times these functions on the host cores: the
reference math of x/fp4x_kernels.py written as torch CPU ops, with each
weight dequantized to fp32 and rounded to the bf16 operand the reference's
kernels feed to their dot (x/fp4x_kernels.py:23, :92, :129, :170, :322),
then an fp32 matmul and the output cast.  tests/test_oracle_torch_cpu.py
checks every function against the numpy oracle: dequantized operands bit for
bit, sums within fp32 summation-order error.
"""
import os

import torch

E2M1 = torch.tensor([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], dtype=torch.float32)
ORDER = (0, 2, 1, 3)


def host_threads():
    """Threads for the CPU baseline: the process's CPU affinity, capped by
    OMP_NUM_THREADS when it is set."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    return min(n, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else n


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def bf16_operand(w):
    return w.to(torch.bfloat16).float()


# ----------------------------------------------------------------- dequant (fp32)
def deq_mx8(w_u8, s_u8):
    """e4m3(w) * 2^(s - 127)  [x/fp4x_kernels.py:22, :261-267]"""
    n, k = w_u8.shape
    w = w_u8.view(torch.float8_e4m3fn).float().view(n, k // 32, 32)
    return (w * torch.exp2(s_u8.float() - 127)[..., None]).view(n, k)


def deq_w8(q, s):
    """q * s per 64 (fp32 or fp16 scales)  [x/fp4x_kernels.py:126-128]"""
    n, k = q.shape
    return (q.float().view(n, k // 64, 64) * s.float()[..., None]).view(n, k)


def deq_w6(L, H, S):
    """((lo | hi << 4) - 32) * S per 32, lo from L (low nibble = even k), the
    high bit pairs of H in the order (0, 2, 1, 3)  [x/fp4x_kernels.py:160-169]"""
    n = L.shape[0]
    lo = torch.stack([L & 15, L >> 4], -1).view(n, -1).int()
    hp = torch.stack([(H >> (2 * j)) & 3 for j in (0, 2, 1, 3)], -1).view(n, -1).int()
    code = (lo | (hp << 4)) - 32
    k = code.shape[1]
    return (code.float().view(n, k // 32, 32) * S.float()[..., None]).view(n, k)


def deq_nv4(P, S_u8):
    """e2m1(P) * e4m3(S) per 16 (the operand before the global scale)  [x/fp4x_kernels.py:85-92]"""
    n = P.shape[0]
    v = torch.stack([E2M1[(P & 15).long()], E2M1[(P >> 4).long()]], -1).view(n, -1)
    k = v.shape[1]
    return (v.view(n, k // 16, 16) * S_u8.view(torch.float8_e4m3fn).float()[..., None]).view(n, k)


def deq_int2(P, S):
    """(code - 1.5) * s per group, element j of a 4-group in bit pair ORDER[j]  [x/fp4x_kernels.py:317-321]"""
    n = P.shape[0]
    code = torch.stack([(P >> (2 * ORDER[j])) & 3 for j in range(4)], -1).view(n, -1).float() - 1.5
    k = code.shape[1]
    g = k // S.shape[1]
    return (code.view(n, k // g, g) * S.float()[..., None]).view(n, k)


# ----------------------------------------------------------------- GEMVs
def gemv(x_bf16, w_op, out_dtype=torch.bfloat16, gs=None):
    """x . w_op^T in fp32 (w_op already the bf16-valued operand), times gs
    after the sum (NVFP4), cast to out_dtype."""
    y = x_bf16.float() @ w_op.T
    if gs is not None:
        y = y * gs
    return y.to(out_dtype)


def mx8_linear(x, w_u8, s_u8, out_dtype=torch.bfloat16):
    return gemv(x, bf16_operand(deq_mx8(w_u8, s_u8)), out_dtype)


def w8_linear(x, q, s, out_dtype=torch.bfloat16):
    return gemv(x, bf16_operand(deq_w8(q, s)), out_dtype)


def w6_linear(x, L, H, S, out_dtype=torch.bfloat16):
    return gemv(x, bf16_operand(deq_w6(L, H, S)), out_dtype)


def nv4_linear(x, P, S_u8, gs, out_dtype=torch.bfloat16):
    return gemv(x, bf16_operand(deq_nv4(P, S_u8)), out_dtype, gs=float(gs))


def int2_logits(x, P, S, out_dtype=torch.float32):
    return gemv(x, bf16_operand(deq_int2(P, S)), out_dtype)


# ----------------------------------------------------------------- mixer
def scaled_silu(d_bf16, lr, hc):
    """bot = bf16(sc * sigmoid(sc)), sc = bf16(d / hc)  [x/fp4x_kernels.py:461-464]"""
    sc = (d_bf16[:, :lr].float() / hc).to(torch.bfloat16).float()
    return (sc * torch.sigmoid(sc)).to(torch.bfloat16)


def gate_mean(nrm_bf16, g_bf16, hc):
    """out = bf16(sum_s bf16(nrm_s * bf16(sigmoid(g_s))) / hc)  [x/fp4x_kernels.py:486-493]"""
    m, n = g_bf16.shape
    h = n // hc
    gate = torch.sigmoid(g_bf16.float()).to(torch.bfloat16).float()
    term = (nrm_bf16[:, :n].float() * gate).to(torch.bfloat16).float().view(m, hc, h)
    tot = term[:, 0]
    for s in range(1, hc):
        tot = tot + term[:, s]
    return (tot / hc).to(torch.bfloat16)


def mixer(x, qd, sd, qu, su, lr, hc):
    """(di, bot, block_input) of one mixer with stream-ordered up rows."""
    di = w8_linear(x, qd, sd)
    bot = scaled_silu(di, lr, hc)
    g = w8_linear(bot, qu, su)
    return di, bot, gate_mean(x, g, hc)


# ----------------------------------------------------------------- fast head
def fast_head(x, P, S, w_u8, s_u8, C):
    """INT2 coarse logits (bf16), their top C rows rescored exactly from the
    MXFP8 head (exact fp32 products, fp32 sum) and written in place."""
    coarse = int2_logits(x, P, S, torch.bfloat16)
    idx = torch.topk(coarse.float(), C, dim=-1).indices
    out = coarse.clone()
    for m in range(x.shape[0]):
        rows = deq_mx8(w_u8[idx[m]], s_u8[idx[m]])
        out[m, idx[m]] = (rows @ x[m].float()).to(torch.bfloat16)
    return out, idx
