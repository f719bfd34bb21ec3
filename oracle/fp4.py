"""FP4 (e2m1) weight codes and e8m0 block scales -- numpy restatement.

Test infrastructure only (see oracle/__init__.py).

Reference files restated here:
* patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:17-30  e2m1_to_codes
* patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:33-41  decode_codes
* patches/tpu-inference-experimental/fused-moe-fp4/
  0901-fused-moe-fp4-codes-routing-oneshot-metadata.patch:84-96  dequant order
* kernels/tpu_inference/layers/common/quantization/e8m0_scale.py:14-40
"""
import numpy as np

from .numerics import round_bf16


def _e2m1_table() -> np.ndarray:
    """OCP MX FP4 E2M1 from its definition: bit3 sign, bits2-1 exponent
    (bias 1), bit0 mantissa; exponent 0 is subnormal (0 or 0.5)."""
    vals = np.zeros(16, np.float32)
    for c in range(16):
        s = -1.0 if c & 8 else 1.0
        e = (c >> 1) & 3
        m = c & 1
        mag = m * 0.5 if e == 0 else (1.0 + m / 2.0) * 2.0 ** (e - 1)
        vals[c] = s * mag
    return vals


E2M1_VALUES = _e2m1_table()


def pack_nibbles(nibbles: np.ndarray) -> np.ndarray:
    """[..., N] values 0..15 -> [..., N/2] bytes, element 2j in the low nibble.

    This is the byte layout of a 4-bit array viewed as uint8 pairs along the
    last dimension (patches/tpu-inference-ext/0103-...:210-221 moves uint4
    weights this way) and of torch ``float4_e2m1fn_x2``.
    """
    nibbles = np.asarray(nibbles, np.uint8)
    assert nibbles.shape[-1] % 2 == 0
    return (nibbles[..., 0::2] & 0xF) | ((nibbles[..., 1::2] & 0xF) << 4)


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """Inverse of ``pack_nibbles``."""
    packed = np.asarray(packed, np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), np.uint8)
    out[..., 0::2] = packed & 0xF
    out[..., 1::2] = packed >> 4
    return out


def e2m1_to_codes(nibbles: np.ndarray) -> np.ndarray:
    """e2m1 nibble c -> uint4 code holding the int4 q = c>=8 ? -(c&7) : c&7.

    patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:17-30.  -0 (c=8)
    becomes +0.
    """
    c = np.asarray(nibbles, np.int16)
    q = np.where(c >= 8, -(c & 7), c & 7)
    return (q & 0xF).astype(np.uint8)


def codes_to_int4(codes: np.ndarray) -> np.ndarray:
    """uint4 code -> its two's complement int4 value (the bitcast at :39)."""
    c = np.asarray(codes, np.int16) & 0xF
    return np.where(c >= 8, c - 16, c).astype(np.int8)


def decode_codes(codes: np.ndarray) -> np.ndarray:
    """uint4 codes -> exact e2m1 values (float32 holding bf16-exact values).

    patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:33-41:
        v = (q + q) - (clip(q, -6, 6) + 0.5 * clip(q, -4, 4))
    Every intermediate is a small multiple of 1/2, so float32 evaluation
    equals the reference's bf16 evaluation bit for bit.
    """
    q = codes_to_int4(codes).astype(np.float32)
    return (q + q) - (np.clip(q, -6, 6) + np.float32(0.5) * np.clip(q, -4, 4))


def e8m0_encode(scale: np.ndarray):
    """f32 scale -> (uint8 codes, lossless flag).

    kernels/tpu_inference/layers/common/quantization/e8m0_scale.py:28-34:
    the code is the f32 biased-exponent field; lossless iff sign and
    mantissa bits (mask 0x807FFFFF, :25) are clear and the exponent is not 255.
    """
    bits = np.ascontiguousarray(scale, np.float32).view(np.uint32)
    exp = bits >> 23
    lossless = bool(np.all(((bits & np.uint32(0x807FFFFF)) == 0) & (exp != 255)))
    return exp.astype(np.uint8), lossless


def e8m0_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 codes -> exact f32 scales: bits = code << 23 (code 0 -> +0.0).

    kernels/tpu_inference/layers/common/quantization/e8m0_scale.py:37-40.
    """
    return (np.asarray(codes, np.uint8).astype(np.uint32) << 23).view(np.float32)


def dequant_fp4_block(codes: np.ndarray, scale: np.ndarray, block: int = 32) -> np.ndarray:
    """codes [K, N] uint4 values, scale [K/block, 1, N] f32 -> [K, N] bf16 values.

    Order of 0901-...:84-96 (the order tokamax gmm_v2 uses for blocks smaller
    than the MXU): decode to bf16, cast the scale to bf16, multiply in bf16.
    """
    k, n = codes.shape
    w = decode_codes(codes).reshape(k // block, block, n)
    s = round_bf16(np.asarray(scale, np.float32).reshape(k // block, 1, n))
    return round_bf16(w * s).reshape(k, n)
