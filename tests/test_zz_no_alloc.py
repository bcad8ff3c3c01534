"""fp4x_int2_topk_noalloc (the fast head's coarse stage with a static device
workspace, for callers that cannot allocate) called through the C ABI: its
coarse logits and top-C indices equal fp4x_int2_topk's with a caller
workspace bit for bit, on two calls in a row, the second smaller (fewer rows
and a shorter head, over the same static array); a request above the limit is
rejected before anything runs."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _call(L, x, P, S, N, C, coarse, idx):
    m, k = x.shape
    return L.fp4x_int2_topk_noalloc(ctypes.c_void_p(x.data_ptr()), k, ctypes.c_void_p(P.data_ptr()),
                                    ctypes.c_void_p(S.data_ptr()), 2, None, ctypes.c_void_p(coarse.data_ptr()), 0,
                                    coarse.stride(0), m, N, k, k // S.shape[1], C, ctypes.c_void_p(idx.data_ptr()), 0,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_int2_topk_noalloc_matches_workspace_path(gpu):
    import _fp4x
    import fp4x_kernels as F
    L = _fp4x.lib()
    assert L.fp4x_int2_topk_noalloc_limit() == 1 << 20
    g = torch.Generator(device=gpu).manual_seed(123)
    for V, M, C in ((248320, 16, 512), (65197, 3, 64)):
        K = 2560
        w = torch.randn((V, K), generator=g, device=gpu) * 0.02
        w[torch.randperm(V, generator=g, device=gpu)[:64]] *= 4
        P, S = F.quantize_int2(w, group=16)
        del w
        x = torch.randn((M, K), generator=g, device=gpu).to(torch.bfloat16)
        ld = -(-V // 8) * 8
        coarse = torch.empty((M, ld), dtype=torch.bfloat16, device=gpu)
        idx = torch.empty((M, C), dtype=torch.int64, device=gpu)
        rc = _call(L, x, P, S, V, C, coarse, idx)
        assert rc == _fp4x.OK, L.fp4x_last_error()
        want_c, want_i = F.int2_topk(x, P, S, V, C)
        torch.cuda.synchronize()
        assert torch.equal(coarse[:, :V].view(torch.int16), want_c.view(torch.int16)), (V, M)
        assert torch.equal(idx, want_i), (V, M)
    # 17 rows of a 2^20-element head need more than the static array: rejected, nothing launched
    rc = L.fp4x_int2_topk_noalloc(None, 2560, None, None, 2, None, None, 0, 1 << 20, 17, 1 << 20, 2560, 16, 64, None,
                                  0, None)
    assert rc == _fp4x.ERR_ARG and b"static workspace" in L.fp4x_last_error()
