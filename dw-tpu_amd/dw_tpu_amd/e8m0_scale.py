"""uint8 exponent storage for power-of-two f32 scales (MOE_SCALE_E8M0).

Mirrors kernels/tpu_inference/layers/common/quantization/e8m0_scale.py:14-40:
a code is the f32 biased-exponent field; code c in 1..254 stands for
2**(c - 127) and code 0 for +0.0.  These are load-time bit operations on
device tensors; the fp4 kernels consume the uint8 codes directly (no per-call
widening to f32).
"""
import torch

_NON_E8M0_BITS = 0x807FFFFF  # sign + mantissa bits must be clear (e8m0_scale.py:25)


def e8m0_encode(scale: torch.Tensor):
    """f32 scale -> (uint8 codes, lossless flag as a 0-d bool tensor)."""
    bits = scale.to(torch.float32).contiguous().view(torch.int32)
    exp = (bits >> 23) & 0xFF
    lossless = torch.all(((bits & _NON_E8M0_BITS) == 0) & (exp != 255))
    return exp.to(torch.uint8), lossless


def e8m0_decode(codes: torch.Tensor) -> torch.Tensor:
    """uint8 codes -> the exact f32 scales they encode."""
    return (codes.to(torch.int32) << 23).view(torch.float32)
