"""gmm_wrapper and the load-time fp4 weight conversion of the MoE GMM path.

Mirrors:
* ``gmm_wrapper`` -- patches/tpu-inference/0001-dsv4-v6e-enablement.patch:214-233
  with the scale widening of patches/tpu-inference-ext/0401-moe-bf16-scales.patch:52-65
  and 0403-moe-e8m0-scales.patch:64-73 (here the kernel reads bf16 / f32 /
  uint8 scales itself, so nothing is widened per call).
* ``fp4_weight_to_codes`` -- patches/tpu-inference/0001-...:276-300: convert
  stored fp4 expert weights once at load time so the per-call gmm streams
  them directly.
"""
import torch

from .gmm_v2 import Fp4Weight, gmm_v2, prepack_fp4


def fp4_weight_to_codes(weight: torch.Tensor, weight_scale: torch.Tensor,
                        rhs_fp4_codes: bool = False, gate_up: bool = False) -> Fp4Weight:
    """Stored fp4 expert weight [E, K, N/2] (+ block scales) -> ``Fp4Weight``.

    The reference re-encodes e2m1 to uint4 codes here (exact); this package
    also relayouts into the kernel's K-major tiles (exact, same bytes).
    ``gate_up``: a [w1 | w3] weight that gmm1 runs with the fused activation.
    """
    if isinstance(weight, Fp4Weight):
        return weight
    return prepack_fp4(weight, weight_scale, rhs_fp4_codes=rhs_fp4_codes, gate_up=gate_up)


def gmm_wrapper(lhs, rhs, rhs_scale, rhs_bias, group_sizes, group_offset, fuse_act=None,
                preferred_element_type=None):
    """gmm_v2 with zero_initialize=False, as the MoE GMM path calls it.

    ``rhs`` is an ``Fp4Weight`` from ``fp4_weight_to_codes`` (then
    ``rhs_scale`` is None), or packed fp4 bytes with their scales.
    """
    if isinstance(rhs, Fp4Weight):
        rhs_fp4_codes = False
    else:
        # uint8 rhs stands for the reference's uint4 code storage; a float4
        # dtype holds raw e2m1 values.
        rhs_fp4_codes = rhs.dtype == torch.uint8
    return gmm_v2(lhs=lhs,
                  rhs=rhs,
                  group_sizes=group_sizes,
                  rhs_scale=rhs_scale,
                  rhs_bias=rhs_bias,
                  group_offset=group_offset,
                  zero_initialize=False,
                  fuse_act=fuse_act,
                  preferred_element_type=preferred_element_type,
                  rhs_fp4_codes=rhs_fp4_codes)
