"""Checkpoint weight formats -> inputs of the hot path, on the GPU (load time).

* ``mxfp4_requant``: an MXFP4 expert checkpoint (OCP MX e2m1 + ue8m0 per 32
  along K, stored [E, N, K/32, 16] + [E, N, K/32]) -> e2m1 codes
  [E, K, N/2] and e8m0 scale codes [E, K/32, 1, N], requantized at block 32
  with power-of-two scales (exact) and checked to be e8m0-encodable -- the
  reference's quantize_tensor(..., power_of_two_scale=True) at block 32
  (patches/tpu-inference/0001-dsv4-v6e-enablement.patch:338-349, :558-562)
  followed by e8m0_encode (e8m0_scale.py:28-35).  ``load_mxfp4_moe_weight``
  chains it with ``fp4_weight_to_codes`` (0001-...:276-300, :305-313).
* ``fp8_block_requant``: an FP8 weight with 128 x 128 block scales
  (DeepSeek: e4m3 [N, K], f32 [N/128, K/128]) -> e4m3 [K, N] and
  power-of-two f32 scales [K/128, 1, N], the dense fp8 kernel's format
  (0001-...:499-512).

Both run one kernel (dwm_mxfp4_requant / dwm_fp8_block_requant) and read
back a two-word status, so they synchronise the stream once.
"""
from dataclasses import dataclass

import torch

from . import _lib
from .fused_moe_gmm import fp4_weight_to_codes


@dataclass
class RequantStatus:
    """Group counts a requantization reported (a group is one 32- or 128-deep
    K-block of one column)."""
    inexact_groups: int     # MXFP4: scale not e8m0-encodable; FP8: values not reproduced
    nonfinite_groups: int   # groups holding a NaN or an infinity

    @property
    def exact(self) -> bool:
        return self.inexact_groups == 0 and self.nonfinite_groups == 0


def _status(st: torch.Tensor) -> RequantStatus:
    v = st.cpu().tolist()
    return RequantStatus(int(v[0]), int(v[1]))


def mxfp4_requant(blocks: torch.Tensor, scales: torch.Tensor, w13_interleave: bool = False):
    """MXFP4 checkpoint tensors -> (codes [E, K, N/2] uint8, scale codes
    [E, K/32, 1, N] uint8, ``RequantStatus``).

    blocks: uint8 [E, N, K/32, 16] or [E, N, K/2] (e2m1 two per byte along K,
    low nibble first); scales: uint8 [E, N, K/32] ue8m0.  ``w13_interleave``:
    the checkpoint's columns alternate w1, w3 and are written [w1 | w3].
    """
    _lib.require_cuda(blocks, scales)
    if blocks.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise ValueError(f"mxfp4_requant: blocks and scales must be uint8, got {blocks.dtype}, {scales.dtype}")
    if blocks.dim() == 4:
        if blocks.shape[-1] != 16:
            raise ValueError(f"mxfp4_requant: blocks must be [E, N, K/32, 16], got {tuple(blocks.shape)}")
        blocks = blocks.reshape(blocks.shape[0], blocks.shape[1], -1)
    if blocks.dim() != 3:
        raise ValueError(f"mxfp4_requant: blocks must be [E, N, K/2], got {tuple(blocks.shape)}")
    e, n, kh = blocks.shape
    k = 2 * kh
    if tuple(scales.shape) != (e, n, k // 32) or k % 32:
        raise ValueError(f"mxfp4_requant: scales {tuple(scales.shape)} do not match blocks [E={e}, N={n}, K={k}]")
    blocks = blocks.contiguous()
    scales = scales.contiguous()
    dev = blocks.device
    codes = torch.empty((e, k, n // 2), dtype=torch.uint8, device=dev)
    scode = torch.empty((e, k // 32, 1, n), dtype=torch.uint8, device=dev)
    st = torch.empty(2, dtype=torch.int32, device=dev)
    _lib.call("dwm_mxfp4_requant", _lib.ptr(blocks), _lib.ptr(scales), e, n, k, 1 if w13_interleave else 0,
              _lib.ptr(codes), _lib.ptr(scode), _lib.ptr(st), _lib.stream_handle(dev))
    return codes, scode, _status(st)


def load_mxfp4_moe_weight(blocks: torch.Tensor, scales: torch.Tensor, w13_interleave: bool = False,
                          gate_up: bool = False):
    """MXFP4 checkpoint -> prepacked ``Fp4Weight`` for gmm_v2 / moe_block.

    Raises ValueError when a scale is not e8m0-encodable or a group holds a
    NaN / infinity (the reference keeps such layers' scales in f32, which
    this kernel path does not take)."""
    codes, scode, status = mxfp4_requant(blocks, scales, w13_interleave)
    if not status.exact:
        raise ValueError(f"load_mxfp4_moe_weight: requantization is not lossless ({status})")
    return fp4_weight_to_codes(codes, scode, gate_up=gate_up)


def fp8_block_requant(weight: torch.Tensor, weight_scale: torch.Tensor, input_layout: str = "nk"):
    """FP8 block-scaled weight -> (e4m3 [K, N] uint8, f32 scales [K/128, 1, N],
    ``RequantStatus``).

    weight: e4m3 codes as uint8 or float8_e4m3fn, [N, K] (``input_layout="nk"``,
    the checkpoint's [out, in]) or [K, N] (``"kn"``); weight_scale: f32
    [N/128, K/128] or [K/128, N/128] to match.
    """
    _lib.require_cuda(weight, weight_scale)
    if input_layout not in ("nk", "kn"):
        raise ValueError(f"fp8_block_requant: input_layout must be 'nk' or 'kn', got {input_layout!r}")
    w = weight.view(torch.uint8) if weight.dtype == torch.float8_e4m3fn else weight
    if w.dtype != torch.uint8 or w.dim() != 2:
        raise ValueError(f"fp8_block_requant: weight must be 2-D e4m3 codes, got {weight.dtype} {tuple(weight.shape)}")
    nk = input_layout == "nk"
    n, k = w.shape if nk else (w.shape[1], w.shape[0])
    want = (n // 128, k // 128) if nk else (k // 128, n // 128)
    if weight_scale.dtype != torch.float32 or tuple(weight_scale.shape) != want:
        raise ValueError(f"fp8_block_requant: weight_scale must be f32 {want}, got {weight_scale.dtype} "
                         f"{tuple(weight_scale.shape)}")
    w = w.contiguous()
    sc = weight_scale.contiguous()
    dev = w.device
    w_out = torch.empty((k, n), dtype=torch.uint8, device=dev)
    s_out = torch.empty((k // 128, 1, n), dtype=torch.float32, device=dev)
    st = torch.empty(2, dtype=torch.int32, device=dev)
    _lib.call("dwm_fp8_block_requant", _lib.ptr(w), _lib.ptr(sc), k, n, 1 if nk else 0, _lib.ptr(w_out),
              _lib.ptr(s_out), _lib.ptr(st), _lib.stream_handle(dev))
    return w_out, s_out, _status(st)
