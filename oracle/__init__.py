"""CPU oracle for the MoE expert hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the math of the reference path (dw-tpu's
tokamax gmm_v2 FP4 patch, MoE fast dispatch / combine, e8m0 scales and the
dense FP8 GEMM).  Every function cites the reference file:line it follows.

Who may use it: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, and only to check results against.  The product
package (``dw_tpu_amd``) never imports it; the product path fails loudly when
its HIP library is missing instead of falling back to anything here.

Parity pins (what checks each function against something other than itself):

* ``fp4.E2M1_VALUES`` / ``e2m1_to_codes`` / ``decode_codes``: exhaustive over
  all 16 nibbles against the OCP MX e2m1 definition and torch's
  ``float4_e2m1fn_x2`` byte layout; the reference docstring magnitudes.
* ``fp4.e8m0_encode`` / ``e8m0_decode``: all 256 codes against ``ldexp`` and
  torch ``float8_e8m0fnu``; the lossless predicate on crafted bit patterns.
* ``numerics.E4M3_VALUES`` / ``to_e4m3``: all 256 codes and random values
  against torch ``float8_e4m3fn``.
* ``gmm.gmm``: brute force on tiny shapes, float64 closed form, per-group
  independence, empty groups.  The reference's f32 accumulation order inside
  gmm_v2 is not vendored, so bit-exact gmm OUTPUT parity is unpinned by
  construction; outputs are checked against a stated bf16 error bound and the
  reference's acceptance rule (``gmm.acceptance_policy``).  The ``seq32``
  accumulation it compares with: a pure-Python per-element loop on tiny
  shapes (the same order, bit for bit) and the sequential-summation bound.
* ``moe.dispatch``: brute force and the identities of
  moe_fast_dispatch.py:14-20.
* ``moe.combine``: an explicit per-element Python loop (tiny shapes).
* ``quant.quantize_tensor_pow2``: the reference's own exactness tests
  (patches/tpu-inference/0001-dsv4-v6e-enablement.patch:110-157).
* ``quant.act_quant_ue8m0``: the DeepSeek act_quant reference restated in the
  reference test (0001-...:47-56) on its own cases (amax floor, clip).
* ``dense_fp8.matmul_w8a16`` / ``matmul_w8a8``: float64 closed form and brute
  force on tiny shapes.
* ``moe.route_topk``: numpy brute force; parity unpinned beyond that (the
  reference's routing lives in un-vendored fused_moe_func).
"""
