"""Checkpoint weight formats -> inputs of the hot path -- numpy restatement.

Test infrastructure only (see oracle/__init__.py).

* MXFP4 expert weights (OCP MX: e2m1 codes, two per byte along K, low nibble
  first, and one ue8m0 scale per 32 K-values; the Hugging Face layout
  ``*_blocks`` [E, N, K/32, 16] + ``*_scales`` [E, N, K/32]) become the fp4
  gmm's inputs: e2m1 codes [E, K, N] (packed two per byte along N) and e8m0
  scale codes [E, K/32, 1, N].  The reference dequantizes the checkpoint and
  requantizes it to e2m1 at block 32 with power-of-two scales, which
  reproduces every value exactly
  (patches/tpu-inference/0001-dsv4-v6e-enablement.patch:338-349 for
  ``power_of_two_scale`` in quantize_tensor; the MXFP4 call site passes it
  for block-32 e2m1, 0001-...:558-562; quantize_moe_weights 0001-...:239-268;
  the reference's own check, test_power_of_two_scale_requantizes_mxfp4_exactly
  0001-...:131-157), then stores the f32 scales as e8m0 codes when that is
  lossless (kernels/tpu_inference/layers/common/quantization/e8m0_scale.py:
  28-35; patches/tpu-inference-ext/0403-moe-e8m0-scales.patch:118-128).
  ``w13_interleave`` (even columns w1, odd w3 -> [w1 | w3], the
  quantize_moe_weights docstring 0001-...:247-250) is applied on the way.
* FP8 weights with 128 x 128 block scales (DeepSeek checkpoints: e4m3
  [out, in] = [N, K] and f32 scales [N/128, K/128]) become the dense fp8
  kernel's inputs: e4m3 [K, N] and power-of-two f32 scales [K/128, 1, N]
  (one per 128-deep K-block and column), exact when the block scales are
  powers of two (0001-...:499-512; the reference's test
  test_power_of_two_scale_requantizes_ue8m0_fp8_blocks_exactly 0001-...:110-129).

Edge behaviour the reference leaves undefined is fixed here and in the
kernels alike: a block holding a NaN or an infinity (e8m0 code 255, e4m3 NaN
code, or an f32 overflow of code x scale) is reported as non-finite and
written as codes 0 with scale code 255 (MXFP4) or scale NaN (FP8).  Checkpoint
e8m0 code 0 is 2^-127 (the OCP MX definition).
"""
import numpy as np

from .fp4 import E2M1_VALUES
from .numerics import E4M3_VALUES, to_e4m3
from .quant import to_e2m1

_NON_E8M0_BITS = np.uint32(0x807FFFFF)  # e8m0_scale.py:25


def _pow2_ceil_f32(scale):
    """2^ceil(log2(s)) via frexp, s > 0; s <= 0 unchanged (0001-...:341-347)."""
    s = np.asarray(scale, np.float32)
    mant, exp = np.frexp(s)
    e = np.where(mant == 0.5, exp - 1, exp)
    with np.errstate(over="ignore", under="ignore"):
        p = np.ldexp(np.float32(1.0), e.astype(np.int32)).astype(np.float32)
    return np.where(s > 0, p, s).astype(np.float32)


def _inv_or_zero(scale):
    """1 / scale in f32; a zero scale or an infinite reciprocal multiplies by 0."""
    s = np.asarray(scale, np.float32)
    with np.errstate(divide="ignore", over="ignore"):
        inv = (np.float32(1.0) / np.where(s == 0, np.float32(1.0), s)).astype(np.float32)
    return np.where((s == 0) | np.isinf(inv), np.float32(0.0), inv).astype(np.float32)


def e8m0_scale_f32(codes):
    """Checkpoint ue8m0 codes -> f32 2^(c - 127) (code 0 -> 2^-127, 255 -> NaN)."""
    c = np.asarray(codes, np.int32)
    with np.errstate(under="ignore", over="ignore"):
        v = np.ldexp(np.float32(1.0), c - 127).astype(np.float32)
    return np.where(c == 255, np.float32(np.nan), v).astype(np.float32)


def mxfp4_requant(blocks, scales, w13_interleave: bool = False):
    """MXFP4 checkpoint -> (codes [E, K, N] uint8 nibbles, scale codes
    [E, K/32, N] uint8, lossy block count, non-finite block count).

    blocks: uint8 [E, N, K/2] (byte k/2 holds k even in the low nibble);
    scales: uint8 [E, N, K/32].  Per (n, 32-block): x = e2m1(code) * 2^(s-127)
    in f32, scale = pow2ceil(absmax / 6), code = rne_e2m1(x * (1/scale)),
    scale code = f32 exponent field, lossy when the scale is not a positive
    normal power of two or +0 (the e8m0_encode check).
    """
    blocks = np.asarray(blocks, np.uint8)
    e, n, kh = blocks.shape
    k = 2 * kh
    codes = np.empty((e, n, k), np.uint8)
    codes[..., 0::2] = blocks & 0xF
    codes[..., 1::2] = blocks >> 4
    vals = E2M1_VALUES[codes].astype(np.float32).reshape(e, n, k // 32, 32)
    sc = e8m0_scale_f32(scales)[..., None]
    with np.errstate(over="ignore", invalid="ignore"):
        x = (vals * sc).astype(np.float32)
    finite = np.isfinite(x).all(axis=-1)
    amax = np.where(finite, np.abs(x).max(axis=-1), np.float32(0)).astype(np.float32)
    scale = _pow2_ceil_f32((amax / np.float32(6.0)).astype(np.float32))
    q = (np.where(finite[..., None], x, np.float32(0)) * _inv_or_zero(scale)[..., None]).astype(np.float32)
    qc = to_e2m1(q)
    bits = scale.view(np.uint32)
    sexp = (bits >> 23) & 0xFF
    lossy = ((bits & _NON_E8M0_BITS) != 0) | (sexp == 255)
    qc = np.where(finite[..., None], qc, 0).astype(np.uint8)
    scode = np.where(finite, sexp, 255).astype(np.uint8)
    lossy = lossy & finite
    qc = qc.reshape(e, n, k)
    if w13_interleave:
        order = np.concatenate([np.arange(0, n, 2), np.arange(1, n, 2)])
        qc, scode = qc[:, order], scode[:, order]
    return (np.ascontiguousarray(qc.transpose(0, 2, 1)), np.ascontiguousarray(scode.transpose(0, 2, 1)),
            int(lossy.sum()), int((~finite).sum()))


def mxfp4_dequant_checkpoint(blocks, scales, w13_interleave: bool = False):
    """The checkpoint's f32 values [E, K, N] (after the optional w13 de-interleave)."""
    blocks = np.asarray(blocks, np.uint8)
    e, n, kh = blocks.shape
    codes = np.empty((e, n, 2 * kh), np.uint8)
    codes[..., 0::2] = blocks & 0xF
    codes[..., 1::2] = blocks >> 4
    v = (E2M1_VALUES[codes].astype(np.float32).reshape(e, n, -1, 32) * e8m0_scale_f32(scales)[..., None])
    v = v.reshape(e, n, 2 * kh).astype(np.float32)
    if w13_interleave:
        v = v[:, np.concatenate([np.arange(0, n, 2), np.arange(1, n, 2)])]
    return np.ascontiguousarray(v.transpose(0, 2, 1))


def mxfp4_dequant_requantized(codes, scale_codes):
    """Values of requantized codes [E, K, N] with scale codes [E, K/32, N]
    (code 0 = +0.0, as e8m0_decode)."""
    c = np.asarray(codes, np.uint8)
    s = (np.asarray(scale_codes, np.uint32) << 23).view(np.float32)
    e, k, n = c.shape
    return (E2M1_VALUES[c].astype(np.float32).reshape(e, k // 32, 32, n) * s[:, :, None, :]).reshape(e, k, n)


def fp8_block_requant(w, scale, input_nk: bool = True, block: int = 128):
    """FP8 block-scaled checkpoint -> (e4m3 codes [K, N], f32 scales
    [K/128, N], inexact block count, non-finite block count).

    w: e4m3 codes [N, K] (input_nk) or [K, N]; scale: f32 [N/128, K/128]
    (input_nk) or [K/128, N/128].  Per (128-deep K-block, column):
    x = e4m3(code) * block_scale in f32, s = pow2ceil(absmax / 448),
    code = rne_e4m3(x * (1/s)); inexact when some code * s != x.
    """
    w = np.asarray(w, np.uint8)
    scale = np.asarray(scale, np.float32)
    if input_nk:
        w = w.T
        scale = scale.T
    k, n = w.shape
    bs = np.repeat(np.repeat(scale, block, axis=0), block, axis=1)[:k, :n]
    with np.errstate(over="ignore", invalid="ignore"):
        x = (E4M3_VALUES[w].astype(np.float32) * bs).astype(np.float32).reshape(k // block, block, n)
    finite = np.isfinite(x).all(axis=1)
    amax = np.where(finite, np.abs(x).max(axis=1), np.float32(0)).astype(np.float32)
    s = _pow2_ceil_f32((amax / np.float32(448.0)).astype(np.float32))
    q = (np.where(finite[:, None, :], x, np.float32(0)) * _inv_or_zero(s)[:, None, :]).astype(np.float32)
    qc = to_e4m3(q)
    back = (E4M3_VALUES[qc].astype(np.float32) * s[:, None, :]).astype(np.float32)
    inexact = ((back != x).any(axis=1)) & finite
    qc = np.where(finite[:, None, :], qc, 0).astype(np.uint8).reshape(k, n)
    s = np.where(finite, s, np.float32(np.nan)).astype(np.float32)
    return qc, s, int(inexact.sum()), int((~finite).sum())
