"""Pins of the MX lhs quantizer oracle (oracle.quant.mx_quantize_e4m3) by
checks other than its own formula: the restatement of the reference's
quantize_tensor with power-of-two scales (quantize_tensor_pow2, itself pinned
by the reference's exactness tests), the e4m3 range and rounding bounds, exact
round trips, and the edge cases.  CPU only."""
import numpy as np
import pytest

from oracle import quant
from oracle.numerics import E4M3_VALUES, bf16_bits, bf16_to_f32, round_bf16


def _bf16(x):
    return bf16_to_f32(bf16_bits(np.asarray(x, np.float32)))


@pytest.fixture
def x(rng):
    v = rng.standard_normal((64, 256)).astype(np.float32)
    v *= np.float32(2.0) ** rng.integers(-30, 30, (64, 1)).astype(np.float32)
    return _bf16(v)


def test_matches_reference_quantize_tensor(x):
    """In range, the codes and scales are quantize_tensor(e4m3, x, -1, 32,
    power_of_two_scale=True) (patches/tpu-inference/0001-...:315-350)."""
    codes, sc = quant.mx_quantize_e4m3(x)
    ref_codes, ref_scale = quant.quantize_tensor_pow2(x, "e4m3", axis=-1, block=32)
    assert np.array_equal(codes, ref_codes)
    assert np.array_equal(np.ldexp(1.0, sc.astype(np.int64) - 127).astype(np.float32), ref_scale)


def test_range_and_rounding_bounds(x):
    """Each block's largest |value| / scale lies in (224, 448] (a floor-based
    exponent, as in OCP MX's shared-exponent rule, would exceed 448), and every
    element is within half an e4m3 ulp: 2^-4 relative for normals, 2^-10
    absolute below 2^-6."""
    codes, sc = quant.mx_quantize_e4m3(x)
    scale = np.ldexp(1.0, sc.astype(np.int64) - 127)
    xb = x.reshape(64, 8, 32).astype(np.float64) / scale[..., None]
    amax = np.abs(xb).max(-1)
    assert np.all((amax > 224) & (amax <= 448))
    q = E4M3_VALUES[codes].reshape(64, 8, 32).astype(np.float64)
    err = np.abs(q - xb)
    assert np.all(err <= np.maximum(2.0 ** -4 * np.abs(xb), 2.0 ** -10))


def test_exact_round_trip_of_representable_blocks(rng):
    """Blocks of e4m3 values times 2^s whose largest magnitude lies in
    (224, 448] come back exactly."""
    vals = E4M3_VALUES[:0x7F].astype(np.float32)  # 0 .. 448
    blocks = rng.choice(vals, (40, 32)) * np.where(rng.random((40, 32)) < 0.5, -1, 1).astype(np.float32)
    blocks[:, 0] = rng.choice(vals[vals > 224], 40)
    s = rng.integers(-60, 60, (40, 1))
    x = (blocks * np.ldexp(np.float32(1), s)).astype(np.float32).reshape(4, 320)
    codes, sc = quant.mx_quantize_e4m3(x)
    assert np.array_equal(quant.mx_dequantize(codes, sc), x)
    assert np.array_equal(sc.reshape(40), (s[:, 0] + 127).astype(np.uint8))


def test_edge_blocks():
    x = np.zeros((1, 32 * 6), np.float32)
    x[0, 32:64] = -0.0                          # block 1: all -0
    x[0, 64 + 3] = np.nan                       # block 2: NaN
    x[0, 96 + 9] = -np.inf                      # block 3: inf
    x[0, 128:160] = np.float32(2.0 ** -133) * np.arange(-16, 16)  # block 4: bf16 subnormals
    x[0, 160:192] = np.float32(3.3e38)          # block 5: the bf16 top
    codes, sc = quant.mx_quantize_e4m3(x)
    assert sc.tolist() == [[1, 1, 255, 255, 1, int(np.frexp(np.float32(3.3e38))[1]) - 8 + 127]]
    assert np.all(codes[0, :32] == 0) and np.all(codes[0, 32:64] == 0x80)
    assert np.all(codes[0, 64:128] == 0x7F)
    # subnormal block: exponent clamped to -126, values 2^-7 * i exact in e4m3
    assert np.array_equal(quant.mx_dequantize(codes[:, 128:160], sc[:, 4:5]), x[:, 128:160])
    assert np.all(E4M3_VALUES[codes[0, 160:192]] <= 448)


def test_block_axis_is_the_last():
    """Scaling one 32-block leaves every other block's codes and scales alone
    (a wrong block axis or size would mix them)."""
    rng = np.random.default_rng(5)
    x = _bf16(rng.standard_normal((3, 128)))
    c0, s0 = quant.mx_quantize_e4m3(x)
    y = x.copy()
    y[1, 32:64] *= 1024
    c1, s1 = quant.mx_quantize_e4m3(y)
    mask = np.ones((3, 128), bool)
    mask[1, 32:64] = False
    assert np.array_equal(c0[mask], c1[mask])
    assert np.array_equal(c0[1, 32:64], c1[1, 32:64]) and s1[1, 1] == s0[1, 1] + 10
    smask = np.ones((3, 4), bool)
    smask[1, 1] = False
    assert np.array_equal(s0[smask], s1[smask])


def test_block_max_product_brute_force(rng):
    """gmm.block_max_product against an explicit loop on a tiny ragged case."""
    from oracle import gmm
    gs = np.array([3, 0, 2], np.int32)
    a = rng.standard_normal((5, 64)).astype(np.float32)
    w = rng.standard_normal((3, 64, 4)).astype(np.float32)
    got = gmm.block_max_product(a, w, gs)
    want = np.zeros((5, 4))
    owner = [0, 0, 0, 2, 2]
    for m in range(5):
        for n in range(4):
            for b in range(2):
                want[m, n] += max(abs(float(a[m, k]) * float(w[owner[m], k, n])) for k in range(32 * b, 32 * b + 32))
    assert np.allclose(got, want, rtol=1e-12, atol=0)


# --------------------------------------------------------------- MXFP4 lhs

def test_mx_e2m1_matches_the_reference_quantizer_on_bf16(rng):
    """mx_quantize_e2m1 is quantize_tensor(e2m1, x, -1, 32,
    power_of_two_scale=True) (0001-...:315-350, restated as
    quantize_tensor_pow2 and pinned by the reference's MXFP4 requant test)
    on bf16 inputs across 60 binades, where the exponent clamp is not hit."""
    x = rng.standard_normal((64, 256)).astype(np.float32)
    x *= np.ldexp(np.float32(1), rng.integers(-30, 30, (64, 8))).repeat(32, axis=1).astype(np.float32)
    x = round_bf16(x)
    codes, sc = quant.mx_quantize_e2m1(x)
    ref_codes, ref_scale = quant.quantize_tensor_pow2(x, "e2m1", -1, 32)
    assert np.array_equal(codes, ref_codes)
    assert np.array_equal(np.ldexp(np.float32(1), sc.astype(np.int64) - 127).astype(np.float32), ref_scale)


@pytest.mark.parametrize("v,want", [(6.0, 6.0), (-0.25, -0.0), (0.75, 1.0), (1.25, 1.0), (1.75, 2.0),
                                    (2.5, 2.0), (3.5, 4.0), (5.0, 4.0), (0.5, 0.5), (-3.0, -3.0)])
def test_mx_e2m1_rounds_to_nearest_even(v, want):
    """Within a block whose largest value is 6 (scale 1): e2m1 ties go to the
    even code (0.25 -> 0, 0.75 -> 1, 1.25 -> 1, 1.75 -> 2, 2.5 -> 2, 3.5 -> 4,
    5 -> 4)."""
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 6.0
    x[0, 7] = v
    c, s = quant.mx_quantize_e2m1(x)
    assert s[0, 0] == 127
    got = quant.mx_dequantize_e2m1(c, s)[0, 7]
    assert got == want and np.signbit(got) == np.signbit(np.float32(want))


def test_mx_e2m1_scale_boundaries_and_special_blocks():
    """absmax exactly 6 * 2^e keeps exponent e, one bf16 ulp above takes
    e + 1; an all-zero block gets the clamped exponent -126; a block with a
    NaN or an infinity gets scale code 255."""
    x = np.zeros((5, 32), np.float32)
    x[0, 3] = 6.0 * 2.0 ** 5                       # exactly 6 * 2^5
    x[1, 3] = 6.0 * 2.0 ** 5 * (1 + 2.0 ** -7)     # next bf16 value up
    x[2, 3] = -6.0 * 2.0 ** -20
    x[3, 5] = np.nan
    x[4, 9] = -np.inf
    _, s = quant.mx_quantize_e2m1(x)
    assert [int(v) for v in s[:, 0]] == [132, 133, 107, 255, 255]
    _, z = quant.mx_quantize_e2m1(np.zeros((1, 32), np.float32))
    assert z[0, 0] == 1  # -126 + 127
