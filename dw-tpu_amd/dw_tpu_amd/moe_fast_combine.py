"""MoE combine: weighted top-k gather-reduce back to token order.

Mirrors kernels/tpu_inference/layers/common/moe_fast_combine.py:

    out[t] = round(sum_k f32(x[idx[t * topk + k]]) * f32(w[t, k]))

f32 products, f32 sum over k = 0..topk-1 left to right from +0.0, one rounding
to ``out_dtype``.  ``combine_xla`` (mode 1, :44-54) and ``combine_pallas``
(mode 2, :138-198) compute the same math in the reference; here both run the
one HIP combine kernel, bit-exact to that definition.
"""
import torch

from . import _lib


def _combine(x, indices, topk_weights, topk, out_dtype):
    if x.dim() != 2:
        raise ValueError("combine: x must be [N, H]")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"combine: x must be bfloat16 or float32, got {x.dtype}")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"combine: out_dtype must be bfloat16 or float32, got {out_dtype}")
    num_tokens = topk_weights.shape[0]
    if topk_weights.dim() != 2 or topk_weights.shape[1] != topk:
        raise ValueError("combine: topk_weights must be [T, topk]")
    if indices.numel() != num_tokens * topk:
        raise ValueError("combine: indices must hold T * topk entries")
    w = topk_weights
    if w.dtype not in (torch.bfloat16, torch.float32):
        w = w.to(torch.float32)
    x = x.contiguous()
    w = w.contiguous()
    idx = indices.reshape(-1).to(torch.int32).contiguous()
    dev = _lib.require_cuda(x, idx, w)
    out = torch.empty((num_tokens, x.shape[1]), dtype=out_dtype, device=dev)
    _lib.call("dwm_moe_combine", _lib.ptr(x), _lib.dtype_code(x.dtype), x.shape[0], x.shape[1], _lib.ptr(idx),
              _lib.ptr(w), _lib.dtype_code(w.dtype), num_tokens, topk, _lib.ptr(out),
              _lib.dtype_code(out_dtype), _lib.stream_handle(dev))
    return out


def combine_xla(x, indices, topk_weights, topk, out_dtype=None):
    """Mode 1. x [N, H]; indices [T * topk]; topk_weights [T, topk]."""
    return _combine(x, indices, topk_weights, topk, out_dtype)


def pallas_supported(x, num_tokens, topk, tm=64) -> bool:
    """The combine kernel takes any 2-D bf16 / f32 device tensor."""
    return x.dim() == 2 and x.dtype in (torch.bfloat16, torch.float32) and x.is_cuda


def combine_pallas(x, indices, topk_weights, topk, out_dtype=None, tm=64, interpret=False):
    """Mode 2 (same math and bits as mode 1)."""
    return _combine(x, indices, topk_weights, topk, out_dtype)


def fast_combine(x, indices, topk_weights, topk, mode=2, out_dtype=None):
    """MOE_FAST_COMBINE entry (moe_fast_combine.py:201-207)."""
    return _combine(x, indices, topk_weights, topk, out_dtype)
