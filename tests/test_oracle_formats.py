"""Oracle number codecs pinned against closed forms and torch's dtypes."""
import numpy as np
import torch

from oracle import formats as fm


def test_e4m3_decode_matches_torch_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = fm.e4m3_decode(codes)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert nan.sum() == 2  # 0x7f and 0xff only


def test_e4m3_closed_form_points():
    assert fm.e4m3_decode(0x7E) == 448.0
    assert fm.e4m3_decode(0x01) == 2.0 ** -9
    assert fm.e4m3_decode(0x08) == 2.0 ** -6
    assert fm.e4m3_decode(0x38) == 1.0
    assert fm.e4m3_decode(0xB8) == -1.0


def test_e4m3_encode_matches_torch_cast():
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 50,
        (rng.standard_normal(50000) * 1e-3).astype(np.float32),
        fm.E4M3[:127],                                          # exact points
        (fm.E4M3[1:127] + fm.E4M3[0:126]) / 2,                  # ties between neighbours
        np.array([447.9, 448, 460, 464, 470, 479.9, 480, 500, 1e9, -464, -480, 2 ** -10, 3 * 2 ** -11],
                 np.float32),
    ]).astype(np.float32)
    v = np.concatenate([v, -v])
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = fm.e4m3_encode(v)
    refv, gotv = fm.e4m3_decode(ref), fm.e4m3_decode(got)
    nan = np.isnan(refv)
    assert np.array_equal(np.isnan(gotv), nan)
    assert np.array_equal(gotv[~nan], refv[~nan])


def test_e4m3_saturating_encode():
    v = np.array([500.0, -1e6, 448.0, 470.0], np.float32)
    assert list(fm.e4m3_decode(fm.e4m3_encode(v, saturate=True))) == [448.0, -448.0, 448.0, 448.0]


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.standard_normal(300000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 300000),
                        np.array([np.inf, -np.inf, 0.0, -0.0, 3.4e38, 1e-40, -1e-45], np.float32)]).astype(np.float32)
    # add exact ties: bf16 values + half an ulp
    b = fm.bf16_to_f32(fm.bf16_bits(v[:1000]))
    ties = (b.view(np.uint32) + 0x8000).view(np.float32)
    v = np.concatenate([v, ties])
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = fm.bf16_bits(v)
    assert np.array_equal(got, ref)


def test_fp16_round_matches_torch():
    rng = np.random.default_rng(2)
    v = (rng.standard_normal(100000) * 10.0 ** rng.integers(-8, 5, 100000)).astype(np.float32)
    ref = torch.from_numpy(v).half().float().numpy()
    assert np.array_equal(fm.f16_round(v), ref)


def test_e8m0_and_e2m1_closed_forms():
    e = np.arange(256)
    got = fm.e8m0_to_f32(e)
    assert got[127] == 1.0 and got[128] == 2.0 and got[0] == np.float32(2.0 ** -127)
    assert np.isinf(got[255])
    assert np.array_equal(got[1:255], np.ldexp(np.float32(1), e[1:255] - 127).astype(np.float32))
    lut = [0, .5, 1, 1.5, 2, 3, 4, 6]
    for c in range(16):
        e2, m = (c >> 1) & 3, c & 1
        mag = m * 0.5 if e2 == 0 else (1 + m * 0.5) * 2.0 ** (e2 - 1)
        assert fm.e2m1_decode(c) == (-mag if c & 8 else mag)
        assert abs(fm.e2m1_decode(c)) == lut[c & 7]
