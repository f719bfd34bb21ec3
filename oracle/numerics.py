"""Bit-level numerics shared by the oracle: bf16 rounding and the e4m3 format.

Test infrastructure only (see oracle/__init__.py).
"""
import numpy as np


def bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even.

    NaN inputs map to a quiet NaN with the same sign.  This is the rounding
    every ``.astype(jnp.bfloat16)`` in the reference performs.
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """float32 values rounded to the nearest bf16, returned as float32."""
    return bf16_to_f32(bf16_bits(x))


def _e4m3_table() -> np.ndarray:
    """OCP FP8 E4M3 (fn variant: no inf, S.1111.111 = NaN), from the format
    definition: bias 7, 3 mantissa bits, subnormals at exponent field 0."""
    vals = np.zeros(256, np.float64)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 7
        if e == 15 and m == 7:
            vals[c] = np.nan
        elif e == 0:
            vals[c] = s * (m / 8.0) * 2.0 ** -6
        else:
            vals[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals.astype(np.float32)


E4M3_VALUES = _e4m3_table()
E4M3_MAX = 448.0

_POS_CODES = np.array([c for c in range(0x7F)], np.int64)  # 0x00..0x7E, ascending value
_POS_VALS = E4M3_VALUES[_POS_CODES].astype(np.float64)


def to_e4m3(x) -> np.ndarray:
    """float32 -> e4m3 codes (uint8), round to nearest even.

    Magnitudes above 448 round to 448 while within half an ulp (< 464) and to
    NaN (0x7F / 0xFF) beyond, as the ``fn`` conversion does.
    """
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64).ravel()
    sign = (np.signbit(x).ravel()).astype(np.uint8) << 7
    idx = np.searchsorted(_POS_VALS, a, side="left")
    idx = np.clip(idx, 1, len(_POS_VALS) - 1)
    lo = _POS_VALS[idx - 1]
    hi = _POS_VALS[idx]
    pick_hi = (hi - a < a - lo) | ((hi - a == a - lo) & (_POS_CODES[idx] % 2 == 0))
    code = np.where(pick_hi, _POS_CODES[idx], _POS_CODES[idx - 1])
    code = np.where(a == 0.0, 0, code)
    code = np.where(a >= 464.0, 0x7F, code)  # overflow -> NaN
    code = np.where(np.isnan(a), 0x7F, code)
    return (code.astype(np.uint8) | sign).reshape(x.shape)


def e4m3_to_f32(codes) -> np.ndarray:
    return E4M3_VALUES[np.asarray(codes, dtype=np.uint8)]
