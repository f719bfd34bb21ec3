"""MoE router on the GPU: the producer of ``topk_weights`` / ``topk_ids``.

* ``fused_moe_fp4_routing``: top-k routing "exactly as fused_moe_func"
  (_fused_moe_fp4_routing,
  patches/tpu-inference-experimental/fused-moe-fp4/0901-...:656-687): score
  function (softmax, sigmoid or DeepSeek V4's sqrtsoftplus), hash routing or
  lax.approx_max_k on the scores (MOE_APPROX_TOPK: no bias), top-k on score
  + e_score_correction_bias (weights stay the unbiased scores) or plain
  top-k, optional renormalization, invalid tokens to expert 0 with weight 0,
  cast to ``dtype``.
* ``dedupe_topk`` (0901-...:98-121): makes each token's expert ids distinct
  for precomputed routing.

Both are one kernel each (dwm_route_topk / dwm_dedupe_topk).
"""
import os

import torch

from . import _lib


def _env_flag(name):
    return os.environ.get(name, "").strip().lower() in ("1", "true", "yes", "on")


def fused_moe_fp4_routing(gating_output: torch.Tensor, top_k: int, renormalize: bool, scoring_fn: str,
                          dtype: torch.dtype, extra: dict = None, approx_topk: bool = None,
                          recall_target: float = None):
    """gating_output [T, E] (bf16 or f32) -> (topk_weights [T, top_k] of
    ``dtype``, topk_ids [T, top_k] int32).

    ``extra`` may hold ``hash_based_topk_indices`` (int [T, top_k]),
    ``e_score_correction_bias`` ([E]) and ``num_valid_tokens`` (int or a
    one-element device tensor); they are popped from it, as the reference
    does.

    ``approx_topk`` (default: the MOE_APPROX_TOPK environment variable, off
    when unset) takes the reference's lax.approx_max_k branch
    (0901-...:671-675): it comes after hash routing and before the
    correction bias, so a bias in ``extra`` is popped but not applied.  The
    exact top-k of the scores is returned; it meets every ``recall_target``
    (default MOE_APPROX_TOPK_RECALL_TARGET, else 0.95; accepted in (0, 1]),
    which is read and checked only when that branch is taken.
    """
    extra = {} if extra is None else extra
    hash_ids = extra.pop("hash_based_topk_indices", None)
    bias = extra.pop("e_score_correction_bias", None)
    num_valid = extra.pop("num_valid_tokens", None)
    if approx_topk is None:
        approx_topk = _env_flag("MOE_APPROX_TOPK")
    if approx_topk and hash_ids is None:
        # The recall target is read only in the approx_max_k branch, as in
        # the reference: a malformed value cannot affect the exact path.
        if recall_target is None:
            recall_target = float(os.environ.get("MOE_APPROX_TOPK_RECALL_TARGET", "0.95"))
        if not 0.0 < recall_target <= 1.0:
            raise ValueError(f"recall_target must be in (0, 1], got {recall_target}")
        bias = None  # the approx_max_k branch ranks the unbiased scores
    _lib.require_cuda(gating_output)
    if gating_output.dim() != 2:
        raise ValueError(f"gating_output must be [T, E], got {tuple(gating_output.shape)}")
    if scoring_fn not in _lib.SCORE_FNS:
        raise NotImplementedError(f"scoring_fn {scoring_fn!r} is not supported")
    if dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"routing weights dtype must be bf16 or f32, got {dtype}")
    t, e = gating_output.shape
    dev = gating_output.device
    logits = gating_output.contiguous()
    if logits.dtype not in (torch.bfloat16, torch.float32):
        logits = logits.float()
    if bias is not None:
        bias = bias.to(device=dev, dtype=torch.float32).contiguous()
        if bias.shape != (e,):
            raise ValueError(f"e_score_correction_bias must be [{e}], got {tuple(bias.shape)}")
    if hash_ids is not None:
        hash_ids = hash_ids.to(device=dev, dtype=torch.int32).contiguous()
        if hash_ids.shape != (t, top_k):
            raise ValueError(f"hash_based_topk_indices must be [{t}, {top_k}], got {tuple(hash_ids.shape)}")
    if num_valid is not None and not isinstance(num_valid, torch.Tensor):
        num_valid = torch.tensor([int(num_valid)], dtype=torch.int32, device=dev)
    elif num_valid is not None:
        num_valid = num_valid.to(device=dev, dtype=torch.int32).reshape(1).contiguous()
    w = torch.empty((t, top_k), dtype=dtype, device=dev)
    ids = torch.empty((t, top_k), dtype=torch.int32, device=dev)
    _lib.call("dwm_route_topk", _lib.ptr(logits), _lib.dtype_code(logits.dtype), t, e, int(top_k),
              _lib.SCORE_FNS[scoring_fn], _lib.ptr(bias), _lib.ptr(hash_ids), 1 if renormalize else 0,
              _lib.ptr(num_valid), _lib.ptr(w), _lib.dtype_code(dtype), _lib.ptr(ids), _lib.stream_handle(dev))
    return w, ids


def dedupe_topk(topk_weights: torch.Tensor, topk_ids: torch.Tensor, num_experts: int):
    """(weights [T, k], ids [T, k]) -> (f32 weights, int32 ids) with each
    token's ids distinct; a repeat's weight moves to its first occurrence."""
    _lib.require_cuda(topk_weights, topk_ids)
    if topk_weights.shape != topk_ids.shape or topk_ids.dim() != 2:
        raise ValueError(f"{tuple(topk_weights.shape)=} != {tuple(topk_ids.shape)=} (both [T, k])")
    t, k = topk_ids.shape
    w = topk_weights.to(torch.float32).contiguous()
    ids = topk_ids.to(torch.int32).contiguous()
    w_out = torch.empty_like(w)
    ids_out = torch.empty_like(ids)
    _lib.call("dwm_dedupe_topk", _lib.ptr(w), _lib.ptr(ids), t, k, int(num_experts), _lib.ptr(w_out),
              _lib.ptr(ids_out), _lib.stream_handle(w.device))
    return w_out, ids_out
