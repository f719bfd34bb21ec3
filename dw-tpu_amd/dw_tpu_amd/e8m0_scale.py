"""Power-of-two scales stored as one byte each (the MOE_SCALE_E8M0 format of
kernels/tpu_inference/layers/common/quantization/e8m0_scale.py:14-40).

The byte is the scale's IEEE f32 exponent field.  So byte c (1..254) is
2**(c - 127), byte 0 is +0.0 (a zero-padded block), and converting back is a
shift into the exponent position.  A scale survives the round trip exactly
when it is +0.0 or a positive normal power of two: sign and mantissa bits
clear, exponent not all ones.  Both directions are elementwise bit operations
on torch tensors (load time); the fp4 kernels read the bytes themselves.
"""
import torch

# Bits that must be zero for a scale to be a byte code: the sign and the
# 23 mantissa bits (e8m0_scale.py:25).
_SIGN_AND_MANTISSA = 0x807FFFFF


def e8m0_encode(scale: torch.Tensor):
    """Scales (any float dtype, widened to f32) -> (uint8 exponent bytes,
    0-d bool tensor: True iff every scale decodes back to itself)."""
    word = scale.to(torch.float32).contiguous().view(torch.int32)
    exponent = torch.bitwise_and(torch.bitwise_right_shift(word, 23), 0xFF)
    exact = torch.bitwise_and(word, _SIGN_AND_MANTISSA) == 0
    lossless = torch.all(exact & (exponent != 0xFF))
    return exponent.to(torch.uint8), lossless


def e8m0_decode(codes: torch.Tensor) -> torch.Tensor:
    """uint8 exponent bytes -> the f32 scales they stand for (byte 0: +0.0)."""
    return torch.bitwise_left_shift(codes.to(torch.int32), 23).view(torch.float32)
