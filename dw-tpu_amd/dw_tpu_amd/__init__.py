"""MI355X-native MoE expert hot path: FP4 grouped matmul, dispatch / combine
and the dense FP8 GEMM, behind the reference's (jamesdborin/dw-tpu) call
signatures.  Kernels are hand-written HIP for gfx950 in ``../csrc``, reached
through the C ABI of ``include/dwtpu_moe.h`` (``libdwtpu_moe.so``)."""
from . import _lib
from .checkpoint_formats import RequantStatus, fp8_block_requant, load_mxfp4_moe_weight, mxfp4_requant
from .e8m0_scale import e8m0_decode, e8m0_encode
from .fused_moe_gmm import fp4_weight_to_codes, gmm_wrapper
from .gmm_v2 import (Fp4Weight, MxLhs, decode_codes, e2m1_to_codes, gmm_v2, mx_quantize, needs_fp4_emulation,
                     prepack_fp4)
from .moe_block import MoeBlockGraph, MoeBlockOutputs, moe_block
from .routing import dedupe_topk, fused_moe_fp4_routing
from .moe_fast_combine import combine_pallas, combine_xla, fast_combine
from .moe_fast_dispatch import (Dispatch, dispatch_gather_pallas, fast_dispatch_gather, moe_dispatch,
                                row_gather, sorted_token_indices)

__all__ = [
    "Dispatch", "Fp4Weight", "RequantStatus", "fp8_block_requant", "load_mxfp4_moe_weight", "mxfp4_requant", "combine_pallas", "combine_xla", "decode_codes", "dispatch_gather_pallas",
    "e2m1_to_codes", "e8m0_decode", "e8m0_encode", "fast_combine", "fast_dispatch_gather",
    "MoeBlockGraph", "MoeBlockOutputs", "dedupe_topk", "fused_moe_fp4_routing", "fp4_weight_to_codes", "gmm_v2", "gmm_wrapper", "moe_block", "moe_dispatch",
    "MxLhs", "mx_quantize", "needs_fp4_emulation", "prepack_fp4",
    "row_gather", "sorted_token_indices",
]
