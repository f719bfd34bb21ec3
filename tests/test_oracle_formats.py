"""Pins the oracle's number formats (e2m1 codes, e8m0 scales, e4m3, bf16)
against their definitions, torch's independent implementations and the
reference's own stated values.  CPU only."""
import numpy as np
import pytest
import torch

from oracle import fp4, numerics


def test_e2m1_table_matches_reference_magnitudes():
    # patches/tokamax/0001-...:35-37: magnitudes by code 0 .5 1 1.5 2 3 4 6.
    assert list(fp4.E2M1_VALUES[:8]) == [0, .5, 1, 1.5, 2, 3, 4, 6]
    assert list(fp4.E2M1_VALUES[8:]) == [-0.0, -.5, -1, -1.5, -2, -3, -4, -6]
    assert np.signbit(fp4.E2M1_VALUES[8])


def test_e2m1_table_matches_torch_fp4_bytes():
    # torch float4_e2m1fn_x2 packs element 0 in the low nibble; float4 ->
    # float conversion is not implemented on CPU, so check through the MX
    # e2m1 round trip: every value of the table re-encodes to its own nibble.
    from oracle.quant import to_e2m1
    codes = to_e2m1(fp4.E2M1_VALUES)
    assert list(codes) == list(range(16))
    packed = fp4.pack_nibbles(np.arange(16, dtype=np.uint8))
    assert list(packed) == [0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE]
    assert torch.from_numpy(packed).view(torch.float4_e2m1fn_x2).shape == (8,)


def test_e2m1_to_codes_then_decode_is_exact_for_all_nibbles():
    nib = np.arange(16, dtype=np.uint8)
    codes = fp4.e2m1_to_codes(nib)
    # q = sign * (2*exponent + mantissa): the 3 magnitude bits, signed.
    q = fp4.codes_to_int4(codes)
    assert list(q) == [0, 1, 2, 3, 4, 5, 6, 7, 0, -1, -2, -3, -4, -5, -6, -7]
    v = fp4.decode_codes(codes)
    want = fp4.E2M1_VALUES.copy()
    want[8] = 0.0  # -0 becomes +0 (:21-22)
    assert np.array_equal(v, want)
    assert not np.any(np.signbit(v[v == 0]))


def test_decode_codes_all_sixteen_codes_closed_form():
    # decode_codes on every uint4 code, including 8 (q = -8) which
    # e2m1_to_codes never produces: 2q - (clip(q,-6,6) + clip(q,-4,4)/2).
    codes = np.arange(16, dtype=np.uint8)
    v = fp4.decode_codes(codes)
    for c in range(16):
        q = c - 16 if c >= 8 else c
        want = 2 * q - (min(max(q, -6), 6) + 0.5 * min(max(q, -4), 4))
        assert v[c] == want
    assert v[8] == -8.0


def test_pack_unpack_roundtrip(rng):
    x = rng.integers(0, 16, (3, 5, 64), dtype=np.uint8)
    assert np.array_equal(fp4.unpack_nibbles(fp4.pack_nibbles(x)), x)


def test_e8m0_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    d = fp4.e8m0_decode(codes)
    assert d[0] == 0.0 and not np.signbit(d[0])
    for c in range(1, 255):
        assert d[c] == np.ldexp(np.float32(1), c - 127)
    assert np.isinf(d[255])
    # torch's float8_e8m0fnu agrees on every finite nonzero code.
    t = torch.from_numpy(codes).view(torch.float8_e8m0fnu).to(torch.float32).numpy()
    assert np.array_equal(t[1:255], d[1:255])


def test_e8m0_encode_roundtrip_and_lossless_predicate():
    scales = np.ldexp(np.ones(254, np.float32), np.arange(-126, 128))
    codes, ok = fp4.e8m0_encode(scales)
    assert ok and np.array_equal(fp4.e8m0_decode(codes), scales)
    _, ok0 = fp4.e8m0_encode(np.array([0.0], np.float32))
    assert ok0
    for bad in (np.float32(3.0), np.float32(-2.0), np.float32(np.inf), np.float32(1e-40), np.float32(-0.0)):
        _, ok = fp4.e8m0_encode(np.array([bad], np.float32))
        assert not ok, bad


def test_dequant_exact_for_all_codes_and_config_scales():
    # pow2 x e2m1 is exact in bf16 for exponents in [-4, 2]: the bf16
    # dequant equals the float64 product for every (code, exponent).
    codes = np.tile(np.arange(16, dtype=np.uint8), 32 * 7).reshape(32 * 7, 16)  # [K=224, N=16]
    exps = np.repeat(np.arange(-4, 3), 16).reshape(7, 1, 16)
    scale = np.ldexp(np.float32(1), exps).astype(np.float32)
    w = fp4.dequant_fp4_block(fp4.e2m1_to_codes(codes), scale)
    want = fp4.decode_codes(fp4.e2m1_to_codes(codes)).astype(np.float64).reshape(7, 32, 16) * np.exp2(exps)
    assert np.array_equal(w.astype(np.float64), want.reshape(224, 16))


def test_bf16_rounding_matches_torch(rng):
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 1e3,
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3.4e38, -0.0, np.inf, -np.inf, 1e-40],
                                 np.float32)])
    got = numerics.bf16_bits(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    nan = numerics.bf16_to_f32(numerics.bf16_bits(np.array([np.nan], np.float32)))
    assert np.isnan(nan).all()


def test_e4m3_table_matches_torch():
    t = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    fin = np.isfinite(t)
    assert np.array_equal(numerics.E4M3_VALUES[fin], t[fin])
    assert np.array_equal(np.isnan(numerics.E4M3_VALUES), ~fin)
    assert np.nanmax(numerics.E4M3_VALUES) == 448.0


def test_to_e4m3_matches_torch_rounding(rng):
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 100,
                        rng.standard_normal(2000).astype(np.float32) * 1e-3,
                        numerics.E4M3_VALUES[np.isfinite(numerics.E4M3_VALUES)],
                        np.array([448.0, 449.0, 463.9, -460.0, 0.0, -0.0], np.float32)])
    got = numerics.to_e4m3(x)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    # compare values (both NaN encodings count as equal)
    gv, wv = numerics.E4M3_VALUES[got], numerics.E4M3_VALUES[want]
    assert np.array_equal(np.isnan(gv), np.isnan(wv))
    ok = ~np.isnan(gv)
    assert np.array_equal(gv[ok], wv[ok])
    assert np.array_equal(np.signbit(gv[ok]), np.signbit(wv[ok]))
