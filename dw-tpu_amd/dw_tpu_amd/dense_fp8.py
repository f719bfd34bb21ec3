"""Dense FP8 block-quantised GEMM with the reference's call signatures.

Mirrors kernels/tpu_inference/kernels/experimental/dense_fp8.py:
``matmul`` (:15-76), ``select_tile`` (:115-138) and ``try_dense_fp8``
(:140-163), on MI355X.  W8A16: per 128-row K block, an f32 dot of bf16
activations with e4m3 weights times an f32 scale per (K block, column),
accumulated in f32 and stored as bf16 (the reference's "native" mode).
``matmul_w8a8`` adds the block variant with e4m3 activations.

Weights: ``prepack_fp8`` relayouts a stored e4m3 weight [K, N] once (load
time) into the kernel's K-major chunks and returns an ``Fp8Weight``; raw
weight tensors are prepacked on every call (one extra pass over the weight).
"""
import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from .dense_fp8_tiles import overrides

E4M3 = torch.float8_e4m3fn


@dataclass(frozen=True)
class Fp8Weight:
    """Prepacked e4m3 weight [K, N] (uint8 device tensor in kernel layout)."""
    weight: torch.Tensor
    k: int
    n: int

    @property
    def shape(self):
        return (self.k, self.n)


def prepack_fp8(weight: torch.Tensor) -> Fp8Weight:
    """e4m3 weight [K, N] (float8_e4m3fn or uint8 codes) -> ``Fp8Weight``."""
    if isinstance(weight, Fp8Weight):
        return weight
    if weight.dim() != 2:
        raise ValueError(f"weight must be [K, N], got {tuple(weight.shape)}")
    w = weight.view(torch.uint8) if weight.dtype == E4M3 else weight
    if w.dtype != torch.uint8:
        raise ValueError(f"weight must be float8_e4m3fn or uint8 codes, got {weight.dtype}")
    w = w.contiguous()
    dev = _lib.require_cuda(w)
    k, n = w.shape
    out = torch.empty(k * n, dtype=torch.uint8, device=dev)
    _lib.call("dwm_dense_fp8_prepack", _lib.ptr(w), k, n, _lib.ptr(out), _lib.stream_handle(dev))
    return Fp8Weight(out, k, n)


def _workspace(m, k, n, dev):
    b = ctypes.c_int64(0)
    _lib.call("dwm_dense_fp8_workspace_size", m, k, n, ctypes.byref(b))
    return None if b.value == 0 else torch.empty(b.value, dtype=torch.uint8, device=dev), b.value


def _aligned(t):
    t = t.contiguous()
    return t.clone() if t.data_ptr() % 16 else t


def matmul(x, w, s, *, tn=1024, tk=1024, tm=16, mode="native"):
    """W8A16 dense GEMM: x [M, K] bf16, w [K, N] e4m3 (or ``Fp8Weight``),
    s [K/128, 1, N] f32 -> bf16 [M, N].  The tile arguments of the TPU kernel
    are accepted and ignored; ``mode`` other than "native" is unsupported
    here (the other reference modes are tiling variants or, for "pre", a
    different rounding)."""
    if mode not in ("native", "megablox"):
        raise NotImplementedError(f"dense_fp8 mode {mode!r} is not supported")
    pw = prepack_fp8(w)
    m, k = x.shape
    n = pw.n
    if k != pw.k:
        raise ValueError(f"x K={k} does not match weight K={pw.k}")
    x = _aligned(x)
    sc = s.reshape(k // 128, n).to(torch.float32).contiguous()
    dev = _lib.require_cuda(x, pw.weight, sc)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    ws, wsb = _workspace(m, k, n, dev)
    _lib.call("dwm_dense_fp8_w8a16", _lib.ptr(x), m, k, n, _lib.ptr(pw.weight), _lib.ptr(sc), _lib.ptr(out),
              _lib.ptr(ws), wsb, _lib.stream_handle(dev))
    return out


def matmul_w8a8(xq, sx, w, sw):
    """W8A8 block GEMM: xq [M, K] e4m3 with sx [M, K/128] f32; w [K, N] e4m3
    (or ``Fp8Weight``) with 128x128 block scales sw [K/128, N/128] f32 ->
    bf16 [M, N]."""
    pw = prepack_fp8(w)
    xq = xq.view(torch.uint8) if xq.dtype == E4M3 else xq
    m, k = xq.shape
    n = pw.n
    if k != pw.k or tuple(sx.shape) != (m, k // 128) or tuple(sw.shape) != (k // 128, n // 128):
        raise ValueError("matmul_w8a8: shapes of xq, sx, w, sw do not match")
    xq = _aligned(xq)
    sx = sx.to(torch.float32).contiguous()
    sw = sw.to(torch.float32).contiguous()
    dev = _lib.require_cuda(xq, sx, pw.weight, sw)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    ws, wsb = _workspace(m, k, n, dev)
    _lib.call("dwm_dense_fp8_w8a8", _lib.ptr(xq), _lib.ptr(sx), m, k, n, _lib.ptr(pw.weight), _lib.ptr(sw),
              _lib.ptr(out), _lib.ptr(ws), wsb, _lib.stream_handle(dev))
    return out


def select_tile(m, k, n):
    """(mode, tm, tk, tn) of the kernel for an M x K x N problem, or None.

    A valid entry of the tile-override table wins (``baseline`` entries
    return None, keeping the caller's path); otherwise any K % 128 == 0,
    N % 16 == 0 problem is supported and the tiles describe the HIP kernel's
    own choice (16/64/128 rows, 64/128 columns, full 128-deep K steps).
    """
    table = overrides()
    if (m, k, n) in table:
        return table[m, k, n]
    if k % 128 or n % 16 or m < 1:
        return None
    tm = 16 if m <= 16 else (64 if m <= 64 else 128)
    tn = 64 if m <= 16 else 128
    return ("native", tm, 128, tn)


def try_dense_fp8(x, weight, scale):
    """Return a supported dense result, or None to retain the caller's fallback."""
    w_dtype = weight.dtype if not isinstance(weight, Fp8Weight) else E4M3
    if x.dtype != torch.bfloat16 or w_dtype != E4M3:
        return None
    if x.dim() != 2 or scale.dtype != torch.float32:
        return None
    if not isinstance(weight, Fp8Weight) and weight.dim() != 2:
        return None
    m, k = x.shape
    wk, n = (weight.k, weight.n) if isinstance(weight, Fp8Weight) else weight.shape
    entry = select_tile(m, k, n)
    if entry is None or wk != k:
        return None
    if tuple(scale.shape) not in ((k // 128, 1, n), (1, k // 128, 1, n)):
        return None
    if not x.is_cuda:
        return None
    try:
        return matmul(x, weight, scale.reshape(k // 128, 1, n))
    except _lib.Unsupported:
        return None
