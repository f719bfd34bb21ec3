"""Pins of oracle/checkpoint.py (checkpoint weight formats) on the CPU.

The reference's own tests for this path state the invariant: requantizing
MX / ue8m0 block data with power-of-two scales reproduces every value
(test_power_of_two_scale_requantizes_mxfp4_exactly and
test_power_of_two_scale_requantizes_ue8m0_fp8_blocks_exactly,
patches/tpu-inference/0001-dsv4-v6e-enablement.patch:110-157); those
inputs are restated here with numpy's generator.  The closed form of the
block-32 e2m1 requantization (a block whose largest magnitude is v moves
its codes up by k = 3, 2, 2, 1, 1, 0, 0 binades for v = .5, 1, 1.5, 2, 3,
4, 6 and its scale down by k) pins the codes themselves.
"""
import numpy as np
import pytest

from oracle import checkpoint as C
from oracle.fp4 import E2M1_VALUES
from oracle.numerics import E4M3_VALUES
from oracle.quant import to_e2m1


def _pack_k(codes):
    """[E, N, K] nibbles -> [E, N, K/2] bytes (even k in the low nibble)."""
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)


def test_mxfp4_roundtrip_is_exact_on_reference_style_inputs():
    # Random e2m1 codes + exponents in [-20, 5) per 32 along K (0001-...:133-141).
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, (4, 64, 256), dtype=np.uint8)
    exps = rng.integers(-20, 5, (4, 64, 256 // 32))
    blocks, scales = _pack_k(codes), (exps + 127).astype(np.uint8)
    q, sc, lossy, nonfinite = C.mxfp4_requant(blocks, scales)
    assert lossy == 0 and nonfinite == 0
    np.testing.assert_array_equal(C.mxfp4_dequant_requantized(q, sc), C.mxfp4_dequant_checkpoint(blocks, scales))


def test_mxfp4_absmax_scale_without_pow2_is_lossy():
    # The reference's negative check (0001-...:151-157): a plain absmax / 6
    # scale does not reproduce the same input.
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, (4, 64, 256), dtype=np.uint8)
    exps = rng.integers(-20, 5, (4, 64, 8))
    x = C.mxfp4_dequant_checkpoint(_pack_k(codes), (exps + 127).astype(np.uint8))  # [E, K, N]
    xb = x.reshape(4, 8, 32, 64)
    s = (np.abs(xb).max(axis=2, keepdims=True) / np.float32(6)).astype(np.float32)
    q = E2M1_VALUES[to_e2m1((xb / np.where(s == 0, 1, s)).astype(np.float32))] * s
    assert not np.array_equal(q.reshape(x.shape), x)


@pytest.mark.parametrize("vmax,shift", [(0.5, 3), (1.0, 2), (1.5, 2), (2.0, 1), (3.0, 1), (4.0, 0), (6.0, 0)])
def test_mxfp4_closed_form_per_block_maximum(vmax, shift):
    # Every code of magnitude <= vmax in one block, the block maximum vmax.
    mags = E2M1_VALUES[:8]
    allowed = [c for c in range(16) if mags[c & 7] <= vmax]
    top = [c for c in range(8) if mags[c] == vmax][0]
    rng = np.random.default_rng(int(vmax * 10))
    codes = rng.choice(allowed, size=(1, 4, 64)).astype(np.uint8)
    codes[:, :, 0] = top
    codes[:, :, 32] = top | 8
    for s in (100, 127, 140):
        q, sc, lossy, _ = C.mxfp4_requant(_pack_k(codes), np.full((1, 4, 2), s, np.uint8))
        assert lossy == 0
        assert (sc == s - shift).all()
        want = E2M1_VALUES[codes].astype(np.float64) * 2.0 ** shift
        got = E2M1_VALUES[q.transpose(0, 2, 1)].astype(np.float64)
        np.testing.assert_array_equal(got, want)


def test_mxfp4_edge_cases():
    codes = np.zeros((1, 64, 128), np.uint8)
    scales = np.full((1, 64, 4), 127, np.uint8)
    codes[0, 1, :32] = 3          # 1.5 * 2^(s-127)
    scales[0, 1, 0] = 255         # NaN scale -> non-finite group
    codes[0, 2, :32] = 7          # 6 * 2^127 overflows f32
    scales[0, 2, 0] = 254
    codes[0, 3, :32] = 1          # 0.5 * 2^-127 -> scale 2^-130: not e8m0-encodable
    scales[0, 3, 0] = 0
    codes[0, 4, :32] = 8          # all -0
    q, sc, lossy, nonfinite = C.mxfp4_requant(_pack_k(codes), scales)
    assert nonfinite == 2 and lossy == 1
    assert sc[0, 0, 1] == 255 and (q[0, :32, 1] == 0).all()
    assert sc[0, 0, 2] == 255 and (q[0, :32, 2] == 0).all()
    assert sc[0, 0, 0] == 0 and (q[0, :, 0] == 0).all()     # zero group: scale +0.0 (code 0)
    assert (q[0, :32, 4] == 8).all() and sc[0, 0, 4] == 0   # -0 keeps its sign bit


def test_mxfp4_w13_interleave_moves_odd_columns_to_the_second_half():
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 16, (2, 128, 128), dtype=np.uint8)
    scales = rng.integers(120, 130, (2, 128, 4)).astype(np.uint8)
    q0, s0, _, _ = C.mxfp4_requant(_pack_k(codes), scales)
    q1, s1, _, _ = C.mxfp4_requant(_pack_k(codes), scales, w13_interleave=True)
    np.testing.assert_array_equal(q1[:, :, :64], q0[:, :, 0::2])
    np.testing.assert_array_equal(q1[:, :, 64:], q0[:, :, 1::2])
    np.testing.assert_array_equal(s1[:, :, 64:], s0[:, :, 1::2])


def test_fp8_block_requant_exact_on_reference_style_inputs():
    # e4m3 weight [in=512, out=384], 128 x 128 blocks with scales 2^[-12, 0)
    # (0001-...:112-125), requantized to 1 x 128 along the contracting dim.
    rng = np.random.default_rng(1)
    w = rng.standard_normal((512, 384)).astype(np.float32)
    from oracle.numerics import to_e4m3
    wc = to_e4m3(w)
    exps = rng.integers(-12, 0, (4, 3))
    scale = np.ldexp(np.float32(1), exps).astype(np.float32)
    qc, s, inexact, nonfinite = C.fp8_block_requant(wc, scale, input_nk=False)
    assert inexact == 0 and nonfinite == 0
    orig = E4M3_VALUES[wc] * np.repeat(np.repeat(scale, 128, 0), 128, 1)
    back = E4M3_VALUES[qc] * np.repeat(s, 128, 0)
    np.testing.assert_array_equal(back, orig)
    # Scales are powers of two no larger than the block's.
    assert (np.frexp(s)[0] == 0.5).all()
    # [N, K] input gives the same result.
    qc2, s2, _, _ = C.fp8_block_requant(wc.T.copy(), scale.T.copy(), input_nk=True)
    np.testing.assert_array_equal(qc2, qc)
    np.testing.assert_array_equal(s2, s)


def test_fp8_block_requant_flags_non_pow2_and_nan_blocks():
    rng = np.random.default_rng(2)
    from oracle.numerics import to_e4m3
    wc = to_e4m3(rng.standard_normal((256, 256)).astype(np.float32))
    scale = np.full((2, 2), np.float32(0.01))      # not a power of two: re-rounding
    _, _, inexact, _ = C.fp8_block_requant(wc, scale, input_nk=False)
    assert inexact > 0
    wc[5, 7] = 0x7F                                # NaN code: one group non-finite
    _, s, _, nonfinite = C.fp8_block_requant(wc, np.ones((2, 2), np.float32), input_nk=False)
    assert nonfinite == 1 and np.isnan(s[0, 7])
