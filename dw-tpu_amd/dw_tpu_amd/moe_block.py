"""The routed-expert block around the FP4 gmm: dispatch, gmm1 (reading the
dispatched rows of ``hidden`` itself: the row gather fused into its loads)
with the fused ``silu_and_mul_with_clamp`` activation, gmm2 and the
routing-weighted combine -- the local (one-GPU) body of the reference's
``moe_gmm_local`` (patches/tpu-inference-ext/0103-...:77-78 for gmm1 with the
activation, 0106-...:239-250 for gmm2 and its f32 variant) with the fast
dispatch / combine of moe_fast_dispatch.py:188-194 and
moe_fast_combine.py:201-207.

Rounding points follow the reference: gmm1 accumulates in f32 and the
activation of the accumulators is rounded once to bf16 (fused-moe-fp4
0901-...:420-423); gmm2 accumulates in f32 and rounds once (0901-...:446-449)
or stays f32 (``f32_reduce``, 0106-...:243-250); the combine sums in f32 in
top-k order and rounds once (moe_fast_combine.py:44-54).

With ``lhs_quant_dtype=torch.float8_e4m3fn`` (or float4_e2m1fn) both gmm
run in the MX mode (gmm_v2.py): ``hidden`` is quantized once, [T, H] before the gather (the
blocks run along each row, so gmm1 reads exactly the quantized rows of the
gathered copy), and gmm2 quantizes the activation.
"""
from dataclasses import dataclass

import torch

from . import _trace
from .gmm_v2 import Fp4Weight, _mx_format, gmm_v2, mx_quantize
from .moe_fast_combine import fast_combine
from .moe_fast_dispatch import moe_dispatch, row_gather


@dataclass
class MoeBlockOutputs:
    """The block's result and its intermediates (device tensors)."""
    out: torch.Tensor       # [T, H] combined
    dispatch: object        # moe_fast_dispatch.Dispatch
    x: torch.Tensor         # [T * topk, H] the rows gmm1 reads (expert order), gathered for inspection
    h: torch.Tensor         # [T * topk, I] activation of gmm1 (bf16)
    y: torch.Tensor         # [T * topk, H] gmm2 output (bf16 or f32)


@_trace.traced("moe_block")
def moe_block(hidden: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, w13: Fp4Weight,
              w2: Fp4Weight, num_experts: int, group_offset=None, f32_reduce: bool = False,
              return_intermediates: bool = False, lhs_quant_dtype=None):
    """hidden [T, H] bf16; topk_ids [T, topk] int32; topk_weights [T, topk]
    f32 or bf16; w13: gate/up weights [E, H, 2I] prepacked with
    ``gate_up=True``; w2: down weights [E, I, H].  Returns [T, H] bf16 (or
    ``MoeBlockOutputs`` with ``return_intermediates``).  ``lhs_quant_dtype``:
    None (the reference's bf16 activations), torch.float8_e4m3fn (the MX
    mode for both gmm) or float4_e2m1fn (MXFP4 activations)."""
    if not w13.gate_up:
        raise ValueError("moe_block: w13 must be prepacked with gate_up=True")
    if w13.k != hidden.shape[1] or w2.k != w13.n // 2 or w2.n != hidden.shape[1]:
        raise ValueError(f"moe_block: shapes do not chain: hidden {tuple(hidden.shape)}, w13 {w13.shape}, w2 {w2.shape}")
    topk = topk_ids.shape[1]
    d = moe_dispatch(topk_ids, num_experts)
    # gmm1 reads hidden[token_indices_sorted] itself (the row gather fused
    # into its loads), the same rows the separate gather would write.
    src = hidden if lhs_quant_dtype is None else mx_quantize(hidden, _mx_format(lhs_quant_dtype))
    h = gmm_v2(src, w13, d.group_sizes, group_offset=group_offset, zero_initialize=False,
               fuse_act="silu_and_mul_with_clamp", lhs_row_indices=d.token_indices_sorted,
               lhs_quant_dtype=lhs_quant_dtype)
    # With a group_offset (an expert-parallel shard) rows of other shards'
    # experts are zeroed before the combine, as the reference does
    # (patches/tpu-inference-ext/0103-...:94-97: 0 * NaN would poison it).
    y = gmm_v2(h, w2, d.group_sizes, group_offset=group_offset, zero_initialize=group_offset is not None,
               preferred_element_type=torch.float32 if f32_reduce else None, lhs_quant_dtype=lhs_quant_dtype)
    out = fast_combine(y, d.topk_argsort_revert_indices, topk_weights, topk, out_dtype=hidden.dtype)
    if return_intermediates:
        return MoeBlockOutputs(out, d, row_gather(hidden, d.token_indices_sorted), h, y)
    return out


class MoeBlockGraph:
    """``moe_block`` captured once into a HIP graph and replayed.

    The reference runs the block as one compiled XLA program; here the
    dispatch, gather, two gmm and combine launches are recorded once (shapes,
    weights and options fixed at construction) and each call replays them
    with one graph launch, so no host work sits between the kernels.  Inputs
    are copied into the graph's own buffers before a replay; the returned
    tensor is the graph's output buffer, overwritten by the next replay.
    Every kernel of the block reads its sizes from device memory (group sizes
    from the dispatch), and none of them allocates or synchronises, so the
    captured work is the eager work.
    """

    def __init__(self, hidden: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, w13: Fp4Weight,
                 w2: Fp4Weight, num_experts: int, group_offset=None, f32_reduce: bool = False,
                 lhs_quant_dtype=None):
        self.hidden = hidden.clone()
        self.topk_ids = topk_ids.to(torch.int32).clone()
        self.topk_weights = topk_weights.clone()
        if isinstance(group_offset, torch.Tensor):
            group_offset = group_offset.clone()
        elif group_offset is not None:
            # an int would become a host-to-device copy inside the capture
            group_offset = torch.tensor([int(group_offset)], dtype=torch.int32, device=hidden.device)
        args = (w13, w2, num_experts)
        kw = dict(group_offset=group_offset, f32_reduce=f32_reduce, lhs_quant_dtype=lhs_quant_dtype)
        self._keep = (w13, w2, group_offset)
        # One eager run on a side stream first (as torch's capture recipe asks).
        side = torch.cuda.Stream(device=hidden.device)
        side.wait_stream(torch.cuda.current_stream(hidden.device))
        with torch.cuda.stream(side):
            moe_block(self.hidden, self.topk_ids, self.topk_weights, *args, **kw)
        torch.cuda.current_stream(hidden.device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = moe_block(self.hidden, self.topk_ids, self.topk_weights, *args, **kw)

    @_trace.traced("moe_block_graph")
    def __call__(self, hidden: torch.Tensor = None, topk_ids: torch.Tensor = None,
                 topk_weights: torch.Tensor = None) -> torch.Tensor:
        """Copies the given inputs (same shapes and dtypes as at construction)
        into the graph's buffers and replays it on the current stream."""
        for src, dst in ((hidden, self.hidden), (topk_ids, self.topk_ids), (topk_weights, self.topk_weights)):
            if src is not None:
                if src.shape != dst.shape:
                    raise ValueError(f"MoeBlockGraph: shape {tuple(src.shape)} != captured {tuple(dst.shape)}")
                dst.copy_(src)
        self.graph.replay()
        return self.out
