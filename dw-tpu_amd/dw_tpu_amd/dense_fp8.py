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

Tiles: ``select_tile`` returns the ``(mode, tm, tk, tn)`` of the launch the
library will make (``dense_fp8_tiles`` maps it to and from the C plan), and
``matmul`` passes a given tile through to the kernel.

Modes: "native", "wide", "flipped" and "megablox" are one arithmetic on
MI355X; "pre" (``matmul_pre``) is the reference's other rounding.
"""
import ctypes
import warnings
from dataclasses import dataclass

import torch

from . import _lib
from .dense_fp8_tiles import DenseTile, default_plan, overrides, plan_to_tile, tile_to_plan

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


def _plan_and_workspace(m, k, n, dev, tile, w8a8):
    """(plan pointer or None, workspace tensor or None, workspace bytes)."""
    plan = None if tile is None else tile_to_plan(tile, max(m, 1), k, n, w8a8)
    b = ctypes.c_int64(0)
    if plan is None:
        _lib.call("dwm_dense_fp8_workspace_size", m, k, n, ctypes.byref(b))
    else:
        _lib.call("dwm_dense_fp8_plan_workspace_size", m, k, n, ctypes.byref(plan), ctypes.byref(b))
    ws = None if b.value == 0 else torch.empty(b.value, dtype=torch.uint8, device=dev)
    return (None if plan is None else ctypes.byref(plan)), ws, b.value


def _aligned(t):
    t = t.contiguous()
    return t.clone() if t.data_ptr() % 16 else t


# Modes of the reference's matmul that compute the "native" arithmetic
# (a per-128-K-block f32 dot, scaled in f32 after the dot) and differ only in
# how the TPU schedules it (dense_fp8.py:1-5, 33-53): "wide" widens the
# weight tile to bf16 first (exact for e4m3), "flipped" computes the dot as
# (w^T x^T)^T.  Here they take the native launches.
SAME_MATH_MODES = {"native": "native", "wide": "native", "flipped": "native", "megablox": "megablox"}


def matmul(x, w, s, *, tn=None, tk=None, tm=None, mode="native", stages=0):
    """W8A16 dense GEMM: x [M, K] bf16, w [K, N] e4m3 (or ``Fp8Weight``),
    s [K/128, 1, N] f32 -> bf16 [M, N].

    mode "native", "wide", "flipped" and "megablox" are the same arithmetic
    (f32 dot per 128-deep K block, times the f32 scale, f32 accumulation);
    "pre" (the reference's other rounding: each weight times its bf16 scale,
    rounded to bf16, before one f32 dot) is ``matmul_pre``.

    With tm, tk and tn left unset the library launches its own plan.  Given,
    they name a launch (``dense_fp8_tiles``: mode "native" = the skinny or
    MFMA kernel, "megablox" = the general tiled kernel; tk = the K depth per
    block; ``stages`` = ring depth).  A tile that names no launch of this
    library (the reference's TPU tiles, e.g. its defaults tm=16, tk=1024,
    tn=1024) gets the library's own plan and a ``UserWarning``: tiles change
    the schedule, never the result.  (An override file that names such a
    tile is rejected when it is read.)"""
    if mode == "pre":
        return matmul_pre(x, w, s)
    if mode not in SAME_MATH_MODES:
        raise NotImplementedError(f"dense_fp8 mode {mode!r} is not supported")
    mode = SAME_MATH_MODES[mode]
    pw = prepack_fp8(w)
    m, k = x.shape
    n = pw.n
    if k != pw.k:
        raise ValueError(f"x K={k} does not match weight K={pw.k}")
    x = _aligned(x)
    sc = s.reshape(k // 128, n).to(torch.float32).contiguous()
    dev = _lib.require_cuda(x, pw.weight, sc)
    tile = None if (tm, tk, tn) == (None, None, None) else DenseTile(mode, tm, tk, tn, stages)
    try:
        plan, ws, wsb = _plan_and_workspace(m, k, n, dev, tile, False)
    except ValueError as exc:
        warnings.warn(f"dense_fp8.matmul: tile {tuple(tile)!r} names no launch of this library ({exc}); "
                      f"using the library's own plan", stacklevel=2)
        plan, ws, wsb = _plan_and_workspace(m, k, n, dev, None, False)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    _lib.call("dwm_dense_fp8_w8a16_plan", _lib.ptr(x), m, k, n, _lib.ptr(pw.weight), _lib.ptr(sc), _lib.ptr(out),
              plan, _lib.ptr(ws), wsb, _lib.stream_handle(dev))
    return out


def matmul_pre(x, w, s):
    """The reference's "pre" mode of the W8A16 GEMM (dense_fp8.py:33-43):
    every e4m3 weight times the bf16-rounded scale of its (128-deep K block,
    column), rounded to bf16 before one f32 dot over K; nothing is scaled
    after the dot.  x [M, K] bf16, w [K, N] e4m3 (or ``Fp8Weight``),
    s [K/128, 1, N] f32 -> bf16 [M, N].  A different rounding from the other
    modes; it runs the general tiled kernel with its own plan."""
    pw = prepack_fp8(w)
    m, k = x.shape
    n = pw.n
    if k != pw.k:
        raise ValueError(f"x K={k} does not match weight K={pw.k}")
    x = _aligned(x)
    sc = s.reshape(k // 128, n).to(torch.float32).contiguous()
    dev = _lib.require_cuda(x, pw.weight, sc)
    b = ctypes.c_int64(0)
    _lib.call("dwm_dense_fp8_workspace_size", m, k, n, ctypes.byref(b))
    ws = None if b.value == 0 else torch.empty(b.value, dtype=torch.uint8, device=dev)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    _lib.call("dwm_dense_fp8_w8a16_pre", _lib.ptr(x), m, k, n, _lib.ptr(pw.weight), _lib.ptr(sc), _lib.ptr(out),
              _lib.ptr(ws), b.value, _lib.stream_handle(dev))
    return out


def matmul_w8a8(xq, sx, w, sw, *, tile=None):
    """W8A8 block GEMM: xq [M, K] e4m3 with sx [M, K/128] f32; w [K, N] e4m3
    (or ``Fp8Weight``) with 128x128 block scales sw [K/128, N/128] f32 ->
    bf16 [M, N].  ``tile``: a ``(mode, tm, tk, tn)`` launch as for ``matmul``
    (None: the library's plan)."""
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
    plan, ws, wsb = _plan_and_workspace(m, k, n, dev, tile, True)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    _lib.call("dwm_dense_fp8_w8a8_plan", _lib.ptr(xq), _lib.ptr(sx), m, k, n, _lib.ptr(pw.weight), _lib.ptr(sw),
              _lib.ptr(out), plan, _lib.ptr(ws), wsb, _lib.stream_handle(dev))
    return out


def last_plan():
    """The ``_lib.DensePlan`` of the last dense GEMM this thread launched."""
    plan = _lib.DensePlan()
    _lib.call("dwm_dense_fp8_last_plan", ctypes.byref(plan))
    return plan


def select_tile(m, k, n):
    """The ``(mode, tm, tk, tn)`` launch for an M x K x N W8A16 problem, or
    None to keep the caller's path.

    An entry of the override file wins (a "baseline" entry gives None);
    otherwise the library's own plan for the shape (``dwm_dense_fp8_plan``),
    i.e. exactly what ``matmul`` launches with no tile given.  Shapes the
    kernels do not take (K % 128, N % 16, M < 1) give None.
    """
    table = overrides()
    if (m, k, n) in table:
        return table[m, k, n]
    if m < 1 or k < 128 or k % 128 or n < 16 or n % 16:
        return None
    return plan_to_tile(default_plan(m, k, n), k)


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
    mode, tm, tk, tn = entry
    try:
        return matmul(x, weight, scale.reshape(k // 128, 1, n), tm=tm, tk=tk, tn=tn, mode=mode,
                      stages=getattr(entry, "stages", 0))
    except _lib.Unsupported:
        return None
