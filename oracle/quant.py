"""Weight/activation (re)quantization formats feeding the hot path -- numpy.

Test infrastructure only (see oracle/__init__.py).

Reference files restated here:
* patches/tpu-inference/0001-dsv4-v6e-enablement.patch:315-350
  (quantize_tensor with power_of_two_scale: 2^ceil(log2(absmax/dtype_max)))
* patches/tpu-inference/0001-dsv4-v6e-enablement.patch:47-56
  (DeepSeek act_quant reference: amax floor 1e-4, pow2 scale, clip +-448)
"""
import numpy as np

from .fp4 import E2M1_VALUES
from .numerics import E4M3_VALUES, to_e4m3

E2M1_MAX = 6.0
E4M3_MAX = 448.0


def pow2_ceil(scale: np.ndarray) -> np.ndarray:
    """2^ceil(log2(s)) for s > 0 computed exactly via frexp (mant in
    [0.5, 1)); s <= 0 passes through (0001-...:339-347)."""
    s = np.asarray(scale, np.float32)
    mant, exp = np.frexp(s)
    e = np.where(mant == 0.5, exp - 1, exp)
    return np.where(s > 0, np.ldexp(np.float32(1.0), e).astype(np.float32), s).astype(np.float32)


def to_e2m1(x: np.ndarray) -> np.ndarray:
    """float32 -> e2m1 nibble (0..15), round to nearest even, saturating at 6."""
    x = np.asarray(x, np.float32)
    mags = E2M1_VALUES[:8].astype(np.float64)  # 0, .5, 1, 1.5, 2, 3, 4, 6
    a = np.minimum(np.abs(x).astype(np.float64), 6.0)
    idx = np.clip(np.searchsorted(mags, a, side="left"), 1, 7)
    lo, hi = mags[idx - 1], mags[idx]
    pick_hi = (hi - a < a - lo) | ((hi - a == a - lo) & (idx % 2 == 0))
    code = np.where(pick_hi, idx, idx - 1)
    code = np.where(a == 0, 0, code)
    return (code | (np.signbit(x).astype(np.int64) << 3)).astype(np.uint8)


def quantize_tensor_pow2(x: np.ndarray, dtype: str, axis: int, block: int):
    """Blockwise quantization along ``axis`` with power-of-two scales.

    0001-...:315-350: scale = absmax / dtype_max rounded up to a power of two;
    q = round(x / scale) in the target format.  Returns (codes, scale) where
    scale has the blocked axis reduced to size len/block (keepdims layout
    [..., nblocks, ...]).
    """
    x = np.asarray(x, np.float32)
    x = np.moveaxis(x, axis, -1)
    shp = x.shape
    xb = x.reshape(shp[:-1] + (shp[-1] // block, block))
    dmax = E2M1_MAX if dtype == "e2m1" else E4M3_MAX
    amax = np.abs(xb).max(axis=-1, keepdims=True)
    scale = pow2_ceil((amax / np.float32(dmax)).astype(np.float32))
    inv = np.where(scale == 0, np.float32(np.inf), np.float32(1.0) / np.where(scale == 0, 1, scale))
    q = xb * np.where(np.isinf(inv), 0, inv).astype(np.float32)
    codes = to_e2m1(q) if dtype == "e2m1" else to_e4m3(q)
    codes = np.moveaxis(codes.reshape(shp), -1, axis)
    scale = np.moveaxis(scale[..., 0], -1, axis)
    return codes, scale


def dequantize(codes: np.ndarray, scale: np.ndarray, dtype: str, axis: int, block: int) -> np.ndarray:
    tab = E2M1_VALUES if dtype == "e2m1" else E4M3_VALUES
    v = np.moveaxis(tab[np.asarray(codes)], axis, -1)
    s = np.moveaxis(np.asarray(scale, np.float32), axis, -1)
    shp = v.shape
    out = v.reshape(shp[:-1] + (shp[-1] // block, block)) * s[..., None]
    return np.moveaxis(out.reshape(shp), -1, axis)


def act_quant_ue8m0(x: np.ndarray, block: int, nope: int) -> np.ndarray:
    """DeepSeek-V4 act_quant(x, block, 'ue8m0', inplace) on x[..., :nope]:
    amax floored at 1e-4, scale 2^ceil(log2(amax/448)), clip to +-448, e4m3
    round, dequantize in place (0001-...:47-56)."""
    out = np.asarray(x, np.float32).copy()
    xb = out[..., :nope].reshape(*x.shape[:-1], nope // block, block)
    amax = np.maximum(np.abs(xb).max(-1, keepdims=True), np.float32(1e-4))
    scale = np.exp2(np.ceil(np.log2(amax / np.float32(448.0)))).astype(np.float32)
    q = np.clip(xb / scale, -448, 448).astype(np.float32)
    q = E4M3_VALUES[to_e4m3(q)]
    out[..., :nope] = (q * scale).reshape(*x.shape[:-1], nope)
    return out


def quantize_fp8_blocks(w: np.ndarray, block=(128, 128)):
    """[K, N] float32 -> (e4m3 codes [K, N], f32 scales [K/bk, N/bn]) with
    scale = block absmax / 448 (not rounded to a power of two)."""
    k, n = w.shape
    bk, bn = block
    wb = np.asarray(w, np.float32).reshape(k // bk, bk, n // bn, bn)
    amax = np.abs(wb).max(axis=(1, 3)).astype(np.float32)
    scale = (amax / np.float32(448.0)).astype(np.float32)
    safe = np.where(scale == 0, np.float32(1), scale)
    q = (wb / safe[:, None, :, None]).astype(np.float32)
    return to_e4m3(q.reshape(k, n)), scale


def quantize_fp8_rows(x: np.ndarray, block: int = 128):
    """[M, K] float32 -> (e4m3 codes [M, K], f32 scales [M, K/block]),
    scale = absmax of each (row, K-block) / 448."""
    m, k = x.shape
    xb = np.asarray(x, np.float32).reshape(m, k // block, block)
    amax = np.abs(xb).max(axis=2).astype(np.float32)
    scale = (amax / np.float32(448.0)).astype(np.float32)
    safe = np.where(scale == 0, np.float32(1), scale)
    return to_e4m3((xb / safe[:, :, None]).reshape(m, k)), scale


MX_BLOCK = 32
MX_MIN_EXP = -126  # scale exponents kept inside e8m0 codes 1..254


def mx_quantize_e4m3(x: np.ndarray, block: int = MX_BLOCK):
    """MX e4m3 activations for the scaled-MFMA grouped matmul
    (gmm_v2(lhs_quant_dtype=float8_e4m3fn)).

    The reference's quantize_tensor(e4m3, x, axis=-1, block,
    power_of_two_scale=True) (patches/tpu-inference/0001-dsv4-v6e-
    enablement.patch:315-350): per block of ``block`` consecutive values
    along the last axis, scale = 2^ceil(log2(absmax / 448)) and codes =
    round-to-nearest-even e4m3 of x / scale (|x / scale| <= 448, so no
    saturation).  The scale is stored as its e8m0 exponent code
    (e8m0_scale.py:28-35: code = exponent + 127), with the exponent kept in
    [-126, 127] (codes 1..254): an all-zero block, or one whose absmax is
    below 448 * 2^-126, gets exponent -126 (its values stay exact or round
    as e4m3 subnormals).  A block holding a NaN or an infinity gets scale
    code 255 (NaN) and element codes 0x7F (NaN).

    The exponent is found without rounding: absmax = mf * 2^ef with mf in
    [0.5, 1) (frexp); absmax <= 448 * 2^e = 0.875 * 2^(9 + e) holds from
    e = ef - 9 when mf <= 0.875, else from e = ef - 8.

    x: float32 values [..., K] with K % block == 0.  Returns (codes uint8
    [..., K], scale codes uint8 [..., K / block]).
    """
    x = np.asarray(x, np.float32)
    shp = x.shape
    xb = x.reshape(shp[:-1] + (shp[-1] // block, block))
    bad = ~np.all(np.isfinite(xb), axis=-1)
    amax = np.where(bad, 0, np.abs(np.where(np.isfinite(xb), xb, 0)).max(axis=-1)).astype(np.float64)
    mf, ef = np.frexp(amax)
    e = np.where(mf > 0.875, ef - 8, ef - 9)
    e = np.where(amax == 0, MX_MIN_EXP, np.maximum(e, MX_MIN_EXP)).astype(np.int64)
    finite = np.where(np.isfinite(xb) & ~bad[..., None], xb, 0).astype(np.float64)
    q = np.ldexp(finite, -e[..., None]).astype(np.float32)  # exact: a power-of-two rescale
    codes = to_e4m3(q)
    codes = np.where(bad[..., None], np.uint8(0x7F), codes).astype(np.uint8)
    scale_codes = np.where(bad, 255, e + 127).astype(np.uint8)
    return codes.reshape(shp), scale_codes


def mx_dequantize(codes: np.ndarray, scale_codes: np.ndarray, block: int = MX_BLOCK) -> np.ndarray:
    """e4m3 codes [..., K] and e8m0 scale codes [..., K / block] -> the
    float32 values they stand for (each e4m3 value times 2^(code - 127),
    exact in f32; scale code 255 gives NaN)."""
    v = E4M3_VALUES[np.asarray(codes, np.uint8)].astype(np.float64)
    sc = np.asarray(scale_codes, np.int64)
    s = np.where(sc == 255, np.nan, np.ldexp(1.0, sc - 127))
    shp = v.shape
    out = v.reshape(shp[:-1] + (shp[-1] // block, block)) * s[..., None]
    return out.reshape(shp).astype(np.float32)


def mx_quantize_e2m1(x: np.ndarray, block: int = MX_BLOCK):
    """MXFP4 activations (gmm_v2(lhs_quant_dtype=float4_e2m1fn)): the
    reference's quantize_tensor(e2m1, x, axis=-1, block,
    power_of_two_scale=True) (patches/tpu-inference/0001-dsv4-v6e-
    enablement.patch:315-350): per block, scale = 2^ceil(log2(absmax / 6))
    and codes = round-to-nearest-even e2m1 of x / scale (|x / scale| <= 6).
    The scale is stored as its e8m0 code (exponent + 127) with the exponent
    kept in [-126, 127]; a block holding a NaN or an infinity gets scale code
    255 and element codes 0.

    The exponent comes from the bits: absmax = mf * 2^ef with mf in [0.5, 1)
    (frexp); absmax <= 6 * 2^e = 0.75 * 2^(e + 3) holds from e = ef - 3 when
    mf <= 0.75, else from e = ef - 2.  (For bf16 inputs this is the same
    power of two as the reference's f32 absmax / 6 rounded up: a bf16
    quotient by 6 lands on a power of two only when it is one exactly.)

    x: float32 [..., K], K % block == 0.  Returns (nibble codes uint8
    [..., K] in 0..15, sign in bit 3; scale codes uint8 [..., K / block]).
    """
    x = np.asarray(x, np.float32)
    shp = x.shape
    xb = x.reshape(shp[:-1] + (shp[-1] // block, block))
    bad = ~np.all(np.isfinite(xb), axis=-1)
    amax = np.where(bad, 0, np.abs(np.where(np.isfinite(xb), xb, 0)).max(axis=-1)).astype(np.float64)
    mf, ef = np.frexp(amax)
    e = np.where(mf > 0.75, ef - 2, ef - 3)
    e = np.where(amax == 0, MX_MIN_EXP, np.maximum(e, MX_MIN_EXP)).astype(np.int64)
    finite = np.where(np.isfinite(xb) & ~bad[..., None], xb, 0).astype(np.float64)
    q = np.ldexp(finite, -e[..., None]).astype(np.float32)  # exact: a power-of-two rescale
    codes = np.where(bad[..., None], np.uint8(0), to_e2m1(q)).astype(np.uint8)
    scale_codes = np.where(bad, 255, e + 127).astype(np.uint8)
    return codes.reshape(shp), scale_codes


def mx_dequantize_e2m1(codes: np.ndarray, scale_codes: np.ndarray, block: int = MX_BLOCK) -> np.ndarray:
    """e2m1 nibble codes [..., K] and e8m0 scale codes [..., K / block] ->
    float32 values (exact; scale code 255 gives NaN)."""
    v = E2M1_VALUES[np.asarray(codes, np.uint8)].astype(np.float64)
    sc = np.asarray(scale_codes, np.int64)
    s = np.where(sc == 255, np.nan, np.ldexp(1.0, sc - 127))
    shp = v.shape
    out = v.reshape(shp[:-1] + (shp[-1] // block, block)) * s[..., None]
    return out.reshape(shp).astype(np.float32)

