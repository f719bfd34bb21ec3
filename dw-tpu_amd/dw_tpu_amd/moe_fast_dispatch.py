"""MoE dispatch: expert-sorted permutation, group sizes and the row gather.

Mirrors kernels/tpu_inference/layers/common/moe_fast_dispatch.py and the
dispatch block of fused_moe_func (patches/tpu-inference-ext/0405-moe-fast-dispatch.patch:70-98):

    topk_argsort_indices = argsort(topk_indices.flatten())      (stable)
    token_indices_sorted = topk_argsort_indices // topk
    group_sizes          = bincount(topk_indices.flatten(), E)
    x                    = hidden[token_indices_sorted]

``moe_dispatch`` produces all index arrays (plus the inverse permutation the
combine consumes) with one counting-sort HIP pipeline, bit-exact to the
stable argsort; ``fast_dispatch_gather`` is the row gather.
"""
import ctypes
from typing import NamedTuple

import torch

from . import _lib


class Dispatch(NamedTuple):
    topk_argsort_indices: torch.Tensor         # int32 [T*topk]
    token_indices_sorted: torch.Tensor         # int32 [T*topk]
    topk_argsort_revert_indices: torch.Tensor  # int32 [T*topk]
    group_sizes: torch.Tensor                  # int32 [E]
    group_offsets: torch.Tensor                # int32 [E + 1]


def moe_dispatch(topk_indices: torch.Tensor, num_experts: int, check: bool = False) -> Dispatch:
    """Dispatch indices for int32 topk_indices [T, topk] (device tensor).

    Ids outside [0, num_experts) sort after all valid ids; with ``check`` the
    call synchronises and raises on such ids.
    """
    if topk_indices.dim() != 2:
        raise ValueError(f"topk_indices must be [T, topk], got {tuple(topk_indices.shape)}")
    ids = topk_indices.to(torch.int32).contiguous()
    dev = _lib.require_cuda(ids)
    t, topk = ids.shape
    n = t * topk
    ws = ctypes.c_int64(0)
    _lib.call("dwm_moe_dispatch_workspace_size", n, num_experts, ctypes.byref(ws))
    workspace = torch.empty(ws.value, dtype=torch.uint8, device=dev)
    perm = torch.empty(n, dtype=torch.int32, device=dev)
    tok = torch.empty(n, dtype=torch.int32, device=dev)
    rev = torch.empty(n, dtype=torch.int32, device=dev)
    gs = torch.empty(num_experts, dtype=torch.int32, device=dev)
    go = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("dwm_moe_dispatch", _lib.ptr(ids), t, topk, num_experts, _lib.ptr(perm), _lib.ptr(tok),
              _lib.ptr(rev), _lib.ptr(gs), _lib.ptr(go), _lib.ptr(flags), _lib.ptr(workspace),
              _lib.stream_handle(dev))
    if check and int(flags.item()):
        raise ValueError(f"topk_indices holds expert ids outside [0, {num_experts})")
    return Dispatch(perm, tok, rev, gs, go)


def sorted_token_indices(topk_argsort_indices: torch.Tensor, topk: int) -> torch.Tensor:
    """== arange(T).repeat(topk)[topk_argsort_indices] (moe_fast_dispatch.py:41-44).

    ``moe_dispatch`` already returns it; this elementwise form serves callers
    that hold only the argsort.
    """
    return torch.div(topk_argsort_indices, topk, rounding_mode="floor").to(torch.int32)


def pallas_supported(hidden: torch.Tensor, num_rows: int, tm: int = 128) -> bool:
    """The row-gather kernel takes any 2-D device tensor (moe_fast_dispatch.py:127-131)."""
    return hidden.dim() == 2 and hidden.is_cuda


def dispatch_gather_pallas(hidden: torch.Tensor, token_indices_sorted: torch.Tensor, tm: int = 128,
                           interpret: bool = False) -> torch.Tensor:
    """hidden[token_indices_sorted], bitwise (moe_fast_dispatch.py:134-185)."""
    return row_gather(hidden, token_indices_sorted)


def row_gather(src: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """src[idx] for a 2-D tensor with JAX gather index semantics (bitwise)."""
    if src.dim() != 2:
        raise ValueError("row_gather: src must be 2-D")
    src = src.contiguous()
    idx = idx.to(torch.int32).contiguous()
    dev = _lib.require_cuda(src, idx)
    rows = idx.numel()
    out = torch.empty((rows, src.shape[1]), dtype=src.dtype, device=dev)
    _lib.call("dwm_row_gather", _lib.ptr(src), src.shape[0], src.shape[1] * src.element_size(),
              _lib.ptr(idx), rows, _lib.ptr(out), _lib.stream_handle(dev))
    return out


def fast_dispatch_gather(hidden: torch.Tensor, topk_argsort_indices: torch.Tensor, topk: int,
                         mode: int = 2) -> torch.Tensor:
    """hidden[arange(T).repeat(topk)[argsort]], bitwise (moe_fast_dispatch.py:188-194).

    One launch (``dwm_dispatch_gather``): the token of each sorted row,
    argsort // topk, is computed inside the gather.  ``mode`` is accepted for
    signature compatibility; both modes run the same HIP gather.
    """
    if hidden.dim() != 2:
        raise ValueError("fast_dispatch_gather: hidden must be 2-D")
    if topk <= 0:
        raise ValueError(f"fast_dispatch_gather: topk must be positive, got {topk}")
    src = hidden.contiguous()
    idx = topk_argsort_indices.to(torch.int32).contiguous().reshape(-1)
    dev = _lib.require_cuda(src, idx)
    rows = idx.numel()
    out = torch.empty((rows, src.shape[1]), dtype=src.dtype, device=dev)
    _lib.call("dwm_dispatch_gather", _lib.ptr(src), src.shape[0], src.shape[1] * src.element_size(),
              _lib.ptr(idx), rows, int(topk), _lib.ptr(out), _lib.stream_handle(dev))
    return out
