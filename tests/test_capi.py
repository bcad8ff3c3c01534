"""libfp4x.so loads, exports every entry point include/fp4x.h declares, and
rejects bad arguments before touching a GPU (no kernel launches here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fp4x.h")
LIB = os.path.join(ROOT, "qwen3.8-flash-next-fp4-local-spark_amd", "libfp4x.so")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(fp4x_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libfp4x.so is not built (run __graft_entry__.build())")
    return ctypes.CDLL(LIB)


def test_header_declares_entry_points():
    names = declared()
    for must in ("fp4x_mx8_linear", "fp4x_w8_linear", "fp4x_w6_linear", "fp4x_nv4_linear", "fp4x_int2_logits",
                 "fp4x_topk_rows", "fp4x_refine_mx8", "fp4x_hc_down", "fp4x_hc_up", "fp4x_hc_scaled_silu",
                 "fp4x_hc_gate_mean", "fp4x_bf16_linear", "fp4x_w8_linear_layers", "fp4x_mx8_dequant",
                 "fp4x_hc_mix", "fp4x_int2_topk", "fp4x_refine_nv4", "fp4x_scatter_draft", "fp4x_quantize",
                 "fp4x_absmax", "fp4x_draft_nv4"):
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version_and_binding(lib):
    import _fp4x
    assert lib.fp4x_abi_version() == _fp4x.ABI_VERSION
    assert set(_fp4x._SIGS) >= set(declared())


def test_layout_query(lib):
    import _fp4x
    assert _fp4x.layout(_fp4x.FMT_MX8, 2560) == (32, 5)     # 160 chunks of 16 fp8
    assert _fp4x.layout(_fp4x.FMT_INT2_F16, 2560) == (8, 5)  # 40 chunks of 64 codes
    assert _fp4x.layout(_fp4x.FMT_W8_F32, 640) == (8, 5)
    assert _fp4x.layout(_fp4x.FMT_W6, 2560) == (16, 5)
    assert _fp4x.layout(_fp4x.FMT_W8_F32, 10240) == (64, 10)
    with pytest.raises(ValueError):
        _fp4x.layout(_fp4x.FMT_MX8, 24)


def test_argument_errors_without_gpu(lib):
    import _fp4x
    L = _fp4x.lib()
    # M > 16, K not a multiple of the group, split without scratch: rejected before any launch
    assert L.fp4x_mx8_linear(None, 2560, None, None, None, 0, 17, 64, 2560, 1, None, None, None) == _fp4x.ERR_ARG
    assert b"M=17" in L.fp4x_last_error()
    assert L.fp4x_w8_linear(None, 100, None, None, 1, None, 0, 1, 8, 100, 1, None, None, None) == _fp4x.ERR_ARG
    assert L.fp4x_w6_linear(None, 2560, None, None, None, None, 0, 1, 8, 2560, 4, None, None, None) == _fp4x.ERR_ARG
    assert L.fp4x_int2_logits(None, 2560, None, None, 2, None, None, 0, 1, 8, 2560, 48, None) == _fp4x.ERR_ARG
    assert L.fp4x_topk_rows(None, 0, 64, 1, 64, 65, None, None, 0, None) == _fp4x.ERR_ARG      # C > V
    assert L.fp4x_topk_rows(None, 2, 64, 1, 64, 8, None, None, 0, None) == _fp4x.ERR_ARG       # fp16 logits
    assert b"bf16 or fp32" in L.fp4x_last_error()
    assert L.fp4x_topk_rows(None, 1, 66, 1, 64, 8, None, None, 0, None) == _fp4x.ERR_ARG       # fp32 rows not 16-byte
    # one u16 maximum per 16-element slice, rows padded to 8 slices
    assert L.fp4x_topk_workspace_size(3, 248320) == 3 * 15520 * 2
    assert L.fp4x_topk_workspace_size(1, 1 << 20) == (1 << 20) // 32 * 2     # 32-element slices past 2^19
    assert L.fp4x_int2_topk(None, 2560, None, None, 2, None, None, 0, 100, 1, 248320, 2560, 16, 512, None, 0, None,
                            0, None) == _fp4x.ERR_ARG                          # coarse stride < N
    assert b"topk" in L.fp4x_last_error()
    assert L.fp4x_hc_up(None, 640, None, None, 1, None, 10240, None, 1, 640, 2560, 4, 3, None) == _fp4x.ERR_ARG
    # the whole mixer: shapes it cannot take reach the down projection's checks (M = 17; split-K without scratch)
    assert L.fp4x_hc_mix(None, 10240, None, None, 1, None, None, 17, 336, 10240, 320, 4, 8, None, None, 0, None,
                         None, None, 10240, None, 2560, 8, None) == _fp4x.ERR_ARG
    assert b"hc_down" in L.fp4x_last_error()
    assert L.fp4x_hc_mix(None, 10240, None, None, 1, None, None, 3, 336, 10240, 320, 4, 8, None, None, 0, None,
                         None, None, 10240, None, 2560, 8, None) == _fp4x.ERR_ARG
    assert b"scratch" in L.fp4x_last_error()
    # the draft head: the NVFP4 rescore needs K % 32 == 0 and rows to gather; the scatter a row stride >= vocab
    assert L.fp4x_refine_nv4(None, None, None, 3, 64, None, None, 1.0, 2500, 100, None) == _fp4x.ERR_ARG
    assert L.fp4x_refine_nv4(None, None, None, 3, 64, None, None, 1.0, 2560, 0, None) == _fp4x.ERR_ARG
    assert b"refine_nv4" in L.fp4x_last_error()
    assert L.fp4x_scatter_draft(None, 100, None, None, None, 10, None, 3, 64, 248320, None) == _fp4x.ERR_ARG
    assert b"scatter_draft" in L.fp4x_last_error()
    # the one-launch rescore + scatter: no weight rows (n_ids = 0), K % 32, C past 2048
    assert L.fp4x_draft_nv4(None, 248320, None, None, None, 0, None, None, 1.0, None, 3, 64, 2560, 248320,
                            None) == _fp4x.ERR_ARG
    assert L.fp4x_draft_nv4(None, 248320, None, None, None, 100, None, None, 1.0, None, 3, 64, 2500, 248320,
                            None) == _fp4x.ERR_ARG
    assert L.fp4x_draft_nv4(None, 248320, None, None, None, 100, None, None, 1.0, None, 3, 2049, 2560, 248320,
                            None) == _fp4x.ERR_ARG
    assert b"draft_nv4" in L.fp4x_last_error()
    # weight preparation: K % 64, the INT2 group, W6 qmax, NVFP4 gs, packed sources without scales
    Q = L.fp4x_quantize
    assert Q(0, None, None, 0.0, 8, 96, 0, 16, 31, 0.0, None, None, None, None) == _fp4x.ERR_ARG
    assert b"K % 64" in L.fp4x_last_error()
    assert Q(0, None, None, 0.0, 8, 128, 3, 128, 31, 0.0, None, None, None, None) == _fp4x.ERR_ARG
    assert Q(0, None, None, 0.0, 8, 128, 1, 16, 40, 0.0, None, None, None, None) == _fp4x.ERR_ARG
    assert Q(0, None, None, 0.0, 8, 128, 2, 16, 31, 0.0, None, None, None, None) == _fp4x.ERR_ARG
    assert b"bad target" in L.fp4x_last_error()
    assert Q(2, None, None, 0.0, 8, 128, 0, 16, 31, 0.0, None, None, None, None) == _fp4x.ERR_ARG
    assert L.fp4x_absmax(1, None, None, 0.0, 8, 100, None, None) == _fp4x.ERR_ARG
    # the CU-holding test kernel: bounded time and LDS
    assert L.fp4x_hold_cus(8, 200000, 160, None, None) == _fp4x.ERR_ARG
    assert L.fp4x_hold_cus(8, 100, 161, None, None) == _fp4x.ERR_ARG
    assert b"hold_cus" in L.fp4x_last_error()
    # empty problems are no-ops
    assert L.fp4x_mx8_linear(None, 2560, None, None, None, 0, 0, 64, 2560, 1, None, None, None) == _fp4x.OK


def test_reload_env(lib, monkeypatch):
    """The path switches are read once; fp4x_reload_env re-reads them
    (no GPU needed: nothing launches)."""
    import _fp4x
    monkeypatch.setenv("FP4X_HC_SPIN_LIMIT", "0")
    _fp4x.reload_env()
    monkeypatch.delenv("FP4X_HC_SPIN_LIMIT")
    _fp4x.reload_env()


def test_splitk_sizes():
    import _fp4x
    part, tick = _fp4x.splitk_sizes(_fp4x.FMT_W8_F32, 3, 640, 10240, 16)
    assert part == 16 * 16 * 640              # one 16-row slot tile per K slice
    assert tick == 640 // 16                  # one ticket per 16-row tile
