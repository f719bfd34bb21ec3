/*
 * dwtpu_moe.h -- C ABI of the MI355X (gfx950) MoE expert hot path.
 *
 * One shared library, libdwtpu_moe.so, built with hipcc for gfx950.  Every
 * entry point takes caller-owned device pointers, plain sizes and a HIP
 * stream handle passed as `void *` (a hipStream_t; NULL = the null stream).
 * Calls are asynchronous on that stream unless stated otherwise, allocate no
 * device memory (scratch comes in through a `workspace` argument sized by a
 * *_workspace_size query) and are reentrant.
 *
 * Return value: DWM_OK, or an error status; dwm_last_error() then returns a
 * thread-local message.  DWM_ERR_UNSUPPORTED means "valid request this
 * library has no kernel for" -- the Python layer maps it to the reference's
 * fail-closed fallback (None), like try_dense_fp8 / pallas_supported.
 * Argument checks run on the host before any launch.
 *
 * References below are to files of the reference (jamesdborin/dw-tpu).
 */
#ifndef DWTPU_MOE_H_
#define DWTPU_MOE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum dwm_status {
  DWM_OK = 0,
  DWM_ERR_INVALID = 1,     /* bad argument (shape, pointer, dtype, value) */
  DWM_ERR_UNSUPPORTED = 2, /* valid but not handled here: caller falls back */
  DWM_ERR_HIP = 3          /* a HIP runtime call failed */
};

enum dwm_dtype {
  DWM_BF16 = 0,
  DWM_F32 = 1,
  DWM_U8 = 2 /* e8m0 exponent codes for scales */
};

/* Activation fused into the grouped matmul's epilogue (gmm_v2 fuse_act):
 * the activations of apply_act_fn
 * (patches/tpu-inference-experimental/fused-moe-fp4/0901-...:57-66) on the
 * f32 accumulators (plus rhs_bias), gate = columns [0, N/2) and up =
 * [N/2, N) of a [w1 | w3] weight; the output has N/2 columns. */
enum dwm_act {
  DWM_ACT_NONE = 0,
  /* silu(min(gate, 10)) * clip(up, -10, 10) (0901-...:60-64). */
  DWM_ACT_SILU_MUL_CLAMP = 1,
  /* silu(gate) * up ("silu"). */
  DWM_ACT_SILU_MUL = 2,
  /* gelu(gate) * up with gelu's tanh form, jax.nn.gelu's default
   * (0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3)))) ("gelu"). */
  DWM_ACT_GELU_TANH_MUL = 3,
  /* GPT-OSS swiglu: g = min(gate, 7), u = clip(up, -7, 7),
   * g * sigmoid(1.702 g) * (u + 1) ("swigluoai"). */
  DWM_ACT_SWIGLUOAI = 4
};

/* Router score functions (apply_scoring_fn, called at
 * patches/tpu-inference-experimental/fused-moe-fp4/0901-...:667). */
enum dwm_score {
  DWM_SCORE_SOFTMAX = 0,      /* exp(x - max) / sum over the experts */
  DWM_SCORE_SIGMOID = 1,      /* 1 / (1 + exp(-x)) */
  DWM_SCORE_SQRTSOFTPLUS = 2  /* sqrt(log(1 + exp(x))), the DeepSeek V4 router score */
};

/* Packed 4-bit weight formats (two per byte, element 2j in the low nibble). */
enum dwm_fp4_format {
  DWM_FP4_E2M1 = 0, /* OCP e2m1 nibbles (torch float4_e2m1fn_x2 bytes) */
  DWM_FP4_CODES = 1 /* gmm_v2 uint4 codes: int4 q = sign*(2*exp+mant) */
};

/* Library version (major*100 + minor). */
int dwm_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *dwm_last_error(void);

/* ---------------------------------------------------------------------- */
/* FP4 weight codes.                                                       */
/* ---------------------------------------------------------------------- */

/* e2m1 nibbles -> gmm_v2 uint4 codes, elementwise over `nbytes` packed bytes.
 * Replaces e2m1_to_codes (patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:17-30)
 * as used by fp4_weight_to_codes (patches/tpu-inference/0001-dsv4-v6e-enablement.patch:276-300). */
int dwm_e2m1_to_codes(const uint8_t *e2m1, uint8_t *codes, int64_t nbytes, void *stream);

/* Decode `n` packed 4-bit values (format DWM_FP4_*) to bf16 bit patterns,
 * each multiplied by the e8m0 scale of its 32-element block along the flat
 * index when `scales` is not NULL (one uint8 code per 32 values).  Bit-exact
 * test hook for decode_codes (patches/tokamax/0001-...:33-41) and the block
 * dequant order of patches/tpu-inference-experimental/fused-moe-fp4/0901-...:84-96.
 * It converts through the same canonical e2m1 nibbles and hardware
 * converter as the gmm kernel.  n must be even.  `flags` (device int32[1])
 * gets bit 0 ORed in for scale code 255 (output NaN) and bit 1 for code 8
 * (q = -8, decoded to -8 * scale although no e2m1 value equals it). */
int dwm_fp4_decode(const uint8_t *packed, int format, int64_t n, const uint8_t *scales,
                   uint16_t *out_bf16, int32_t *flags, void *stream);

/* ---------------------------------------------------------------------- */
/* FP4 grouped matmul (tokamax gmm_v2 with rhs_fp4_codes).                 */
/* ---------------------------------------------------------------------- */

/* Bytes of the load-time weight layout produced by dwm_gmm_fp4_prepack for
 * E experts of a [K, N] fp4 matrix with 32-element e8m0 block scales along K.
 * Requires K % 128 == 0 and N % 16 == 0. */
int dwm_gmm_fp4_prepack_size(int64_t E, int64_t K, int64_t N, int64_t *weight_bytes,
                             int64_t *scale_bytes);

/* One-time relayout of expert weights into the kernel's K-major tiles; the
 * load-time step the reference performs with fp4_weight_to_codes
 * (patches/tpu-inference/0001-...:276-300, shard_moe_weights :302-313).
 *   rhs:   [E, K, N/2] bytes, format DWM_FP4_E2M1 or DWM_FP4_CODES.
 *   scale: [E, K/32, N] (the reference's [E, K/32, 1, N]) of dtype
 *          DWM_U8 (e8m0 codes, e8m0_scale.py:14-40), DWM_F32 or DWM_BF16.
 *          f32/bf16 scales must be powers of two or +0.0 (the lossless
 *          e8m0 subset, e8m0_scale.py:25-34).
 *   flags: device int32[1]; the kernel ORs 1 into it for a scale that is not
 *          an e8m0-representable power of two or +0.0 (including code 255).
 *          The caller zeroes it beforehand and checks it after the stream
 *          synchronises (weight load time).
 * Scale code 0 (+0.0) is kept exact: the block's values become +-0 with
 * the sign of the decoded code, as decode(q) * bf16(0.0) gives. */
int dwm_gmm_fp4_prepack(const uint8_t *rhs, int format, const void *scale, int scale_dtype,
                        int64_t E, int64_t K, int64_t N, uint8_t *weight_out,
                        uint8_t *scale_out, int32_t *flags, void *stream);

/* The same relayout for a gate/up weight [w1 | w3] (the GMM_EP
 * [E, hidden, 2 * inter] layout, patches/tpu-inference-experimental/
 * fused-moe-fp4/0901-...:250-254) that dwm_gmm_fp4 will run with
 * DWM_ACT_SILU_MUL_CLAMP: gate and up columns are interleaved by 32 so each
 * output column's pair is computed together.  Requires N % 64 == 0.  Such
 * weights must be used with the fused activation. */
int dwm_gmm_fp4_prepack_gate_up(const uint8_t *rhs, int format, const void *scale, int scale_dtype,
                                int64_t E, int64_t K, int64_t N, uint8_t *weight_out,
                                uint8_t *scale_out, int32_t *flags, void *stream);

/* dwm_gmm_fp4_prepack (gate_up = 0) or dwm_gmm_fp4_prepack_gate_up
 * (gate_up != 0) from a transposed weight: rhs is [E, N, K/2] bytes, two K
 * values per byte (low nibble = even k), the layout gmm_v2(...,
 * transpose_rhs=True) takes (patches/tokamax/0001-gmm_v2-fp4-emulation-
 * v6e.patch:64-65, :111); scale keeps the [E, K/32, N] layout above.  The
 * prepacked output is the same bytes the untransposed weight gives, so the
 * grouped matmul runs unchanged (the transpose happens once, at load). */
int dwm_gmm_fp4_prepack_transposed(const uint8_t *rhs, int format, const void *scale, int scale_dtype,
                                   int64_t E, int64_t K, int64_t N, int gate_up, uint8_t *weight_out,
                                   uint8_t *scale_out, int32_t *flags, void *stream);

/* Ragged grouped matmul on prepacked weights:
 *   for g in [group_offset, group_offset + E_local):
 *     out[off_g : off_g + size_g] = lhs[off_g : off_g + size_g] @ dequant(rhs[g - group_offset])
 * with off_g the exclusive prefix sum of group_sizes[0..num_groups).  bf16 x
 * bf16 products of the exact dequantised weights, f32 accumulation, output
 * bf16 (round to nearest even) or f32.  Rows outside the local groups are
 * zeroed when zero_init != 0 and left untouched otherwise.
 * Replaces gmm_v2(lhs, rhs, group_sizes, rhs_scale, group_offset,
 * preferred_element_type, zero_initialize, rhs_fp4_codes=True)
 * (patches/tokamax/0001-...:100-151) behind gmm_wrapper
 * (patches/tpu-inference/0001-...:214-233).
 *   lhs:          [M, K] bf16, expert-sorted rows.
 *   group_sizes:  device int32[num_groups].
 *   group_offset: device int32[1] or NULL (= 0).
 *   out_dtype:    DWM_BF16 or DWM_F32 (the MOE_F32_REDUCE variant,
 *                 patches/tpu-inference-ext/0106-...:243-250).
 *   fuse_act:     DWM_ACT_NONE, or a gated DWM_ACT_* with weights from
 *                 dwm_gmm_fp4_prepack_gate_up: out is then [M, N/2], the
 *                 activation of the f32 accumulators rounded once (gmm_v2's
 *                 fuse_act as gmm1 of moe_gmm_local uses it,
 *                 patches/tpu-inference-ext/0103-...:77-78; the
 *                 activations of apply_act_fn, patches/tpu-inference-
 *                 experimental/fused-moe-fp4/0901-...:57-66).
 * Requires K % 128 == 0, N % 16 == 0 (N % 64 == 0 with fuse_act),
 * num_groups <= 1024. */
int dwm_gmm_fp4(const uint16_t *lhs, int64_t M, int64_t K, const uint8_t *weight,
                const uint8_t *scale, const int32_t *group_sizes, int num_groups,
                const int32_t *group_offset, int64_t E_local, int64_t N, void *out,
                int out_dtype, int zero_init, int fuse_act, void *stream);

/* dwm_gmm_fp4 with the dispatch row gather fused into its lhs loads: row r
 * of the grouped operand is lhs[row_idx[r]] (lhs: [lhs_rows, K] bf16, the
 * tokens' hidden states; row_idx: device int32[M], JAX gather index
 * semantics as dwm_row_gather), so
 *   dwm_gmm_fp4_gather(hidden, T, tok_sorted, M, ...)
 * gives the bits of dwm_row_gather(hidden -> x) then dwm_gmm_fp4(x, M, ...)
 * without writing x.  Replaces the gather + gmm1 pair of moe_gmm_local
 * (moe_fast_dispatch.py:188-194 feeding patches/tpu-inference-ext/0103-...:77-78).
 * Requires lhs_rows * K * 2 < 2^32; otherwise as dwm_gmm_fp4. */
int dwm_gmm_fp4_gather(const uint16_t *lhs, int64_t lhs_rows, const int32_t *row_idx, int64_t M, int64_t K,
                       const uint8_t *weight, const uint8_t *scale, const int32_t *group_sizes, int num_groups,
                       const int32_t *group_offset, int64_t E_local, int64_t N, void *out, int out_dtype,
                       int zero_init, int fuse_act, void *stream);

/* The grouped lhs of dwm_gmm_fp4_ex. */
typedef struct dwm_gmm_lhs {
  const void *data;        /* bf16 [rows, K]; e4m3 codes [rows, K] when scale != NULL */
  const uint8_t *scale;    /* NULL, or e8m0 codes [rows, K/32]: the MX mode (dwm_gmm_fp4_mx) */
  int64_t rows;            /* rows of data */
  const int32_t *row_idx;  /* NULL (row r is row r of data; rows == M), or int32 [M]: row r is
                              data[row_idx[r]] (the fused gather, JAX gather semantics) */
} dwm_gmm_lhs;

/* Every form of the grouped matmul in one entry point: the lhs of
 * dwm_gmm_fp4 / dwm_gmm_fp4_gather / dwm_gmm_fp4_mx (by `lhs`), plus
 * rhs_bias: NULL or [E_local, N] of bias_dtype (DWM_F32 or DWM_BF16), in the
 * weight's source column order ([w1 | w3] for gate/up weights), added in f32
 * to every accumulator of the expert's rows before the activation and the
 * output rounding -- gmm_v2's rhs_bias (passed by gmm_wrapper,
 * patches/tpu-inference/0001-dsv4-v6e-enablement.patch:214-233; the
 * reference's MXFP4 MoE carries w13_bias / w2_bias,
 * patches/tpu-inference-ext/0103-...:311-312).  fuse_act: any DWM_ACT_*
 * (the gated ones need weights from dwm_gmm_fp4_prepack_gate_up).  Other
 * arguments and limits as dwm_gmm_fp4. */
int dwm_gmm_fp4_ex(const dwm_gmm_lhs *lhs, int64_t M, int64_t K, const uint8_t *weight, const uint8_t *scale,
                   const void *rhs_bias, int bias_dtype, const int32_t *group_sizes, int num_groups,
                   const int32_t *group_offset, int64_t E_local, int64_t N, void *out, int out_dtype, int zero_init,
                   int fuse_act, void *stream);

/* ---------------------------------------------------------------------- */
/* MX mode: e4m3 activations with e8m0 block-32 scales (scaled MFMA).      */
/* ---------------------------------------------------------------------- */

/* bf16 x [rows, K] -> e4m3 codes [rows, K] and e8m0 scale codes
 * [rows, K/32]: the reference's power-of-two block quantizer
 * quantize_tensor(e4m3, x, axis=-1, 32, power_of_two_scale=True)
 * (patches/tpu-inference/0001-dsv4-v6e-enablement.patch:315-350) applied to
 * the gmm lhs, as gmm_v2 quantizes its lhs for a native low-precision matrix
 * path (lhs_quant_dtype, patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:
 * 89-100).  Per 32-value block: scale 2^e with e the smallest exponent such
 * that absmax <= 448 * 2^e, kept >= -126; codes = e4m3 of x * 2^-e, round to
 * nearest even; scale code = e + 127 (codes 1..254).  A block holding a NaN
 * or infinity gets codes 0x7F (NaN) and scale code 255.  Bit-exact.
 * Requires K % 32 == 0; x 16-byte and codes 8-byte aligned. */
int dwm_mx_quant_e4m3(const uint16_t *x, int64_t rows, int64_t K, uint8_t *codes, uint8_t *scales,
                      void *stream);

/* The grouped matmul of dwm_gmm_fp4 / dwm_gmm_fp4_gather on MX operands:
 * lhs e4m3 codes [lhs_rows, K] with e8m0 scales lhs_scale [lhs_rows, K/32]
 * (dwm_mx_quant_e4m3), the same prepacked weights, one gfx950 scaled MFMA
 * (e4m3 x e2m1, 32x32x64, both block scales in the instruction) per 64-deep
 * K step, f32 accumulation.  Every product e4m3 * 2^a * e2m1 * 2^b is exact;
 * the result differs from dwm_gmm_fp4's by the lhs quantization.  Row r of
 * the grouped operand is row r of lhs, or row row_idx[r] (JAX gather
 * semantics) when row_idx is not NULL (then lhs_rows may differ from M).
 * Other arguments and rules as dwm_gmm_fp4; lhs_rows * K < 2^32; lhs_scale
 * 4-byte aligned.  Stands in for gmm_v2(..., lhs_quant_dtype=float8_e4m3fn)
 * (patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:89-99): the MX
 * quantization (block 32, power-of-two e8m0 scales, dwm_mx_quant_e4m3) is
 * this library's choice, the reference's checkpoint quantizer
 * quantize_tensor(e4m3, x, -1, 32, power_of_two_scale=True); tokamax's own
 * online lhs quantizer is not vendored, so parity with that path is
 * unpinned.  The result is held to this library's stated MX bound. */
int dwm_gmm_fp4_mx(const uint8_t *lhs, const uint8_t *lhs_scale, int64_t lhs_rows, const int32_t *row_idx,
                   int64_t M, int64_t K, const uint8_t *weight, const uint8_t *scale,
                   const int32_t *group_sizes, int num_groups, const int32_t *group_offset, int64_t E_local,
                   int64_t N, void *out, int out_dtype, int zero_init, int fuse_act, void *stream);

/* MXFP4 lhs quantization: bf16 x [rows, K] -> e2m1 codes [rows, K/2] (value
 * 2j in the low nibble of byte j) + e8m0 scale codes [rows, K/32]: per 32
 * values along K the exponent e = the smallest >= -126 with absmax <= 6 *
 * 2^e (the scale 2^ceil(log2(absmax / 6)) of the reference's
 * quantize_tensor(e2m1, x, -1, 32, power_of_two_scale=True),
 * patches/tpu-inference/0001-dsv4-v6e-enablement.patch:315-350), codes the
 * round-to-nearest-even e2m1 of x * 2^-e, scale code e + 127.  A block with a
 * NaN or an infinity gets codes 0 and scale code 255.  K % 32 == 0; x
 * 16-byte and codes 4-byte aligned. */
int dwm_mx_quant_e2m1(const uint16_t *x, int64_t rows, int64_t K, uint8_t *codes, uint8_t *scales,
                      void *stream);

/* dwm_gmm_fp4_mx on an MXFP4 lhs (dwm_mx_quant_e2m1: e2m1 codes [lhs_rows,
 * K/2], e8m0 scales [lhs_rows, K/32]): the gfx950 scaled MFMA with both
 * operands e2m1 (32x32x64, both block scales in the instruction), f32
 * accumulation, with rhs_bias (NULL or [E_local, N], DWM_F32 / DWM_BF16) and
 * fuse_act as dwm_gmm_fp4_ex.  Stands in for gmm_v2(...,
 * lhs_quant_dtype=float4_e2m1fn) (patches/tokamax/0001-gmm_v2-fp4-emulation-
 * v6e.patch:89-99); like the e4m3 MX mode it is this library's choice of
 * lhs quantization, opt-in, lossier than e4m3 (e2m1 keeps two significant
 * bits of each activation), and held to its own stated bound. */
int dwm_gmm_fp4_mxfp4(const uint8_t *lhs, const uint8_t *lhs_scale, int64_t lhs_rows, const int32_t *row_idx,
                      int64_t M, int64_t K, const uint8_t *weight, const uint8_t *scale, const void *rhs_bias,
                      int bias_dtype, const int32_t *group_sizes, int num_groups, const int32_t *group_offset,
                      int64_t E_local, int64_t N, void *out, int out_dtype, int zero_init, int fuse_act,
                      void *stream);

/* ---------------------------------------------------------------------- */
/* MoE dispatch and combine.                                               */
/* ---------------------------------------------------------------------- */

/* Scratch bytes for dwm_moe_dispatch over n = T*topk ids and E experts. */
int dwm_moe_dispatch_workspace_size(int64_t n, int num_experts, int64_t *bytes);

/* Expert-sorted dispatch indices from topk_ids [T, topk] (int32):
 *   perm        = stable argsort(topk_ids.flatten())     (0405-moe-fast-dispatch.patch:73)
 *   tok_sorted  = perm / topk                           (moe_fast_dispatch.py:41-44)
 *   revert      = inverse permutation of perm           (combine indices, moe_fast_combine.py:14-22)
 *   group_sizes = bincount(topk_ids, num_experts)       (0405-...:85-87)
 *   group_offsets (nullable) = [0, cumsum(group_sizes)]  (num_experts + 1 entries)
 * Bit-exact.  Ids outside [0, num_experts) are rejected on the device:
 * `flags` (device int32[1], nullable) gets bit 0 ORed in and such ids are
 * ordered after every valid id. */
int dwm_moe_dispatch(const int32_t *topk_ids, int64_t T, int topk, int num_experts,
                     int32_t *perm, int32_t *tok_sorted, int32_t *revert, int32_t *group_sizes,
                     int32_t *group_offsets, int32_t *flags, void *workspace, void *stream);

/* dwm_moe_dispatch without a workspace argument and without allocating: no
 * counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops).  The
 * chunk counters of batches above 8192 ids live in a 4 MiB device array of
 * the library (one per GPU, held until the process ends), so
 * ceil(T*topk / 1024) * (num_experts + 1) must be <= 2^20 (e.g. T*topk <=
 * 4,177,920 at 256 experts); larger requests return DWM_ERR_UNSUPPORTED
 * before any device work.  Every call on a GPU uses that GPU's one array:
 * calls that overlap on one GPU (on different streams) race and must not be
 * issued.  Results are bit-identical to dwm_moe_dispatch's.  The array's
 * address on a device is looked up (hipGetSymbolAddress) by the first call
 * there with more than 8192 ids; batches of at most 8192 ids never use it.
 * A caller that captures a larger batch into a HIP graph makes one such
 * call on that device before the capture. */
int dwm_moe_dispatch_noalloc(const int32_t *topk_ids, int64_t T, int topk, int num_experts, int32_t *perm,
                             int32_t *tok_sorted, int32_t *revert, int32_t *group_sizes, int32_t *group_offsets,
                             int32_t *flags, void *stream);

/* out[j, :] = src[idx[j], :] for j < rows, bitwise, with JAX gather index
 * semantics (a negative index wraps once, then indices clamp into
 * [0, src_rows)).  Replaces dispatch_gather_pallas / hidden[tok_sorted]
 * (moe_fast_dispatch.py:134-194). */
int dwm_row_gather(const void *src, int64_t src_rows, int64_t row_bytes, const int32_t *idx,
                   int64_t rows, void *out, void *stream);

/* out[j, :] = hidden[argsort[j] // topk, :] for j < rows (floor division,
 * then the JAX gather index semantics of dwm_row_gather), bitwise: the rows
 * of the expert-sorted argsort's tokens in one launch.  Replaces
 * fast_dispatch_gather(hidden, topk_argsort_indices, topk)
 * (moe_fast_dispatch.py:41-44, 188-194). */
int dwm_dispatch_gather(const void *hidden, int64_t T, int64_t row_bytes, const int32_t *argsort, int64_t rows,
                        int topk, void *out, void *stream);

/* out[t] = round(sum_{k=0..topk-1} f32(x[idx[t*topk+k]]) * f32(w[t, k])),
 * summed left to right from +0.0 with separately rounded f32 multiply and
 * add (no FMA), one rounding to out_dtype.  Bit-exact to combine_xla /
 * combine_pallas (moe_fast_combine.py:44-54, 57-122, 201-207).
 *   x: [x_rows, H] of x_dtype (DWM_BF16 / DWM_F32); idx: [T*topk] int32
 *   (JAX gather semantics as dwm_row_gather); w: [T, topk] of w_dtype;
 *   out: [T, H] of out_dtype. */
int dwm_moe_combine(const void *x, int x_dtype, int64_t x_rows, int64_t H, const int32_t *idx,
                    const void *w, int w_dtype, int64_t T, int topk, void *out, int out_dtype,
                    void *stream);

/* ---------------------------------------------------------------------- */
/* Dense FP8 block-quantised GEMM.                                         */
/* ---------------------------------------------------------------------- */

/* One-time relayout of an e4m3 weight [K, N] (row-major, the reference's
 * layout) into the kernel's K-major 2 KiB chunks (16 columns x 128 K).
 * The load-time analogue of storing the FP8 weight for try_dense_fp8
 * (patches/tpu-inference/0006-dense-fp8-gemm.patch:141-176).
 * Requires K % 128 == 0, N % 16 == 0; out holds K*N bytes. */
int dwm_dense_fp8_prepack(const uint8_t *w, int64_t K, int64_t N, uint8_t *out, void *stream);

/* Workspace bytes the W8A16, W8A8 and "pre" entry points below need for
 * M x K x N with their default plans (split-K partials for small M; 0 when
 * none). */
int dwm_dense_fp8_workspace_size(int64_t M, int64_t K, int64_t N, int64_t *bytes);

/* W8A16: out[M, N] bf16 = sum over 128-row K blocks kb of
 * dot(x[:, kb], w[kb, :]) (f32) * s[kb, n] (f32), f32 accumulation.
 * Replaces dense_fp8.matmul / try_dense_fp8
 * (kernels/tpu_inference/kernels/experimental/dense_fp8.py:15-76, 140-163).
 *   x: [M, K] bf16; w: prepacked e4m3; s: [K/128, N] f32 (the reference's
 *   [K/128, 1, N]). */
int dwm_dense_fp8_w8a16(const uint16_t *x, int64_t M, int64_t K, int64_t N, const uint8_t *w,
                        const float *s, uint16_t *out, void *workspace, int64_t workspace_bytes,
                        void *stream);

/* The reference's "pre" rounding of the W8A16 GEMM: out[M, N] bf16 =
 * sum_k x[m, k] * bf16(w[k, n] * bf16(s[k/128, n])), f32 accumulation: every
 * weight is multiplied by its bf16-rounded scale and rounded to bf16 (round
 * to nearest even) before the dot, and nothing is scaled after it.  Replaces
 * dense_fp8.matmul(..., mode='pre')
 * (kernels/tpu_inference/kernels/experimental/dense_fp8.py:33-43).  Same
 * arguments as dwm_dense_fp8_w8a16; it runs the general tiled kernel
 * (DWM_DENSE_TILED) with that kernel's default plan for the shape. */
int dwm_dense_fp8_w8a16_pre(const uint16_t *x, int64_t M, int64_t K, int64_t N, const uint8_t *w,
                            const float *s, uint16_t *out, void *workspace, int64_t workspace_bytes,
                            void *stream);

/* W8A8 block variant: out[m, n] = sum_kb sx[m, kb] * sw[kb, n/128] *
 * dot(xq[m, kb], wq[kb, n]), bf16 output.  No reference kernel (the
 * reference's dense path is W8A16); the per-token-per-128 activation and
 * 128x128 weight block scales follow DeepSeek's block FP8 format.
 *   xq: [M, K] e4m3; sx: [M, K/128] f32; w: prepacked e4m3;
 *   sw: [K/128, N/128] f32.  Requires N % 128 == 0. */
int dwm_dense_fp8_w8a8(const uint8_t *xq, const float *sx, int64_t M, int64_t K, int64_t N,
                       const uint8_t *w, const float *sw, uint16_t *out, void *workspace,
                       int64_t workspace_bytes, void *stream);

/* Launch plans of the dense GEMM: what the reference's tile selection
 * (select_tile, _TUNED, _DECODE_TILES and the tile-override table,
 * kernels/tpu_inference/kernels/experimental/dense_fp8.py:80-138,
 * dense_fp8_tiles.py:11-58) and matmul's tm/tk/tn (dense_fp8.py:15-76) choose
 * there, expressed in this library's kernels. */
enum dwm_dense_kernel {
  /* M <= 16: one block per 16 columns; its 16 waves split K (ksplit = 16)
   * and add their f32 partial sums in wave order; register ring depth 2. */
  DWM_DENSE_SKINNY = 1,
  /* tile_m x 128 tiles (tile_m 128 or 256), 32x32 MFMA (bf16 for W8A16, fp8
   * for W8A8) fed by an LDS ring of `stages` K steps.  Needs M > 16 and
   * N % 128 == 0. */
  DWM_DENSE_MFMA = 2,
  /* General tiles for any N % 16 == 0: 16 x 64, 64 x 128 or 128 x 128,
   * 16x16x32 bf16 MFMA, double-buffered LDS (stages = 2). */
  DWM_DENSE_TILED = 3
};

typedef struct dwm_dense_plan {
  int32_t kernel; /* enum dwm_dense_kernel */
  int32_t tile_m; /* output rows per block */
  int32_t tile_n; /* output columns per block */
  int32_t ksplit; /* K runs per output tile (blocks, or the skinny kernel's waves),
                     each ceil(K/128 / ksplit) 128-deep blocks, none empty; their
                     f32 partials are added in run order and rounded once */
  int32_t stages; /* ring depth (LDS stages, or the skinny kernel's register ring) */
} dwm_dense_plan;

/* The plan the library launches by default for M x K x N (w8a8 != 0: the
 * W8A8 variant).  M = 0 plans as M = 1. */
int dwm_dense_fp8_plan(int64_t M, int64_t K, int64_t N, int w8a8, dwm_dense_plan *plan);

/* DWM_OK if `plan` is a configuration this library has a kernel for at
 * M x K x N, else DWM_ERR_UNSUPPORTED with the reason in dwm_last_error(). */
int dwm_dense_fp8_plan_check(int64_t M, int64_t K, int64_t N, int w8a8, const dwm_dense_plan *plan);

/* Workspace bytes `plan` needs (ksplit > 1 outside the skinny kernel:
 * ksplit * M * N f32 partials). */
int dwm_dense_fp8_plan_workspace_size(int64_t M, int64_t K, int64_t N, const dwm_dense_plan *plan,
                                      int64_t *bytes);

/* dwm_dense_fp8_w8a16 / dwm_dense_fp8_w8a8 with an explicit launch plan
 * (NULL: the default plan).  Every plan gives the same products and the same
 * 128-K partial sums; only the order in which K runs are added differs. */
int dwm_dense_fp8_w8a16_plan(const uint16_t *x, int64_t M, int64_t K, int64_t N, const uint8_t *w,
                             const float *s, uint16_t *out, const dwm_dense_plan *plan, void *workspace,
                             int64_t workspace_bytes, void *stream);
int dwm_dense_fp8_w8a8_plan(const uint8_t *xq, const float *sx, int64_t M, int64_t K, int64_t N,
                            const uint8_t *w, const float *sw, uint16_t *out, const dwm_dense_plan *plan,
                            void *workspace, int64_t workspace_bytes, void *stream);

/* The plan of the last dense GEMM this thread launched (all zero before the
 * first), so callers and tests can see which configuration ran. */
int dwm_dense_fp8_last_plan(dwm_dense_plan *plan);

/* ---------------------------------------------------------------------- */
/* Checkpoint weight formats (load time).                                  */
/* ---------------------------------------------------------------------- */

/* MXFP4 expert weights (OCP MX: e2m1 codes two per byte along K, low nibble
 * first; one ue8m0 scale per 32 K-values, code 0 = 2^-127, 255 = NaN) ->
 * the fp4 gmm's inputs, requantized at block 32 with power-of-two scales
 * and the scales stored as e8m0 codes (code 0 = +0.0).  Replaces the
 * reference's load path: quantize_tensor(e2m1, dequantized checkpoint, K,
 * 32, power_of_two_scale=True) (patches/tpu-inference/
 * 0001-dsv4-v6e-enablement.patch:338-349, called at :558-562 from
 * quantize_moe_weights :239-268) followed by e8m0_encode
 * (kernels/tpu_inference/layers/common/quantization/e8m0_scale.py:28-35,
 * patches/tpu-inference-ext/0403-moe-e8m0-scales.patch:118-128).
 *   blocks:  [E, N, K/2] bytes; scales: [E, N, K/32] e8m0 codes.
 *   w13_interleave: columns stored w1, w3, w1, w3, ... are written
 *     [w1 | w3] (quantize_moe_weights' w13_interleave).
 *   codes_out: [E, K, N/2] bytes (e2m1 two per byte along N, the input of
 *     dwm_gmm_fp4_prepack); scale_codes_out: [E, K/32, N] e8m0 codes.
 *   status: device int32[2], set by the call: [0] = groups whose scale is
 *     not e8m0-encodable (e8m0_encode's lossless flag is status[0] == 0),
 *     [1] = groups holding a NaN or infinity (written as codes 0, scale
 *     code 255).
 * Requires K % 128 == 0, N % 64 == 0 (N % 128 == 0 with w13_interleave). */
int dwm_mxfp4_requant(const uint8_t *blocks, const uint8_t *scales, int64_t E, int64_t N, int64_t K,
                      int w13_interleave, uint8_t *codes_out, uint8_t *scale_codes_out, int32_t *status,
                      void *stream);

/* FP8 weights with 128 x 128 block scales (DeepSeek checkpoints) -> e4m3
 * [K, N] with power-of-two f32 scales per (128-deep K-block, column), the
 * layout of dwm_dense_fp8_prepack / the reference's [K/128, 1, N] scales.
 * Exact when the block scales are powers of two (ue8m0).  Replaces the
 * reference's requantization to 1 x 128 K-blocks with power_of_two_scale
 * (patches/tpu-inference/0001-dsv4-v6e-enablement.patch:499-512, checked by
 * its test at :110-129).
 *   w: e4m3 [N, K] (input_nk != 0, the checkpoint's [out, in]) or [K, N];
 *   scale: f32 [N/128, K/128] (input_nk) or [K/128, N/128].
 *   w_out: [K, N] e4m3; scale_out: [K/128, N] f32.
 *   status: device int32[2], set by the call: [0] = (K-block, column) groups
 *     the requantization does not reproduce exactly, [1] = groups holding a
 *     NaN or infinity (written as codes 0, scale NaN).
 * Requires K % 128 == 0, N % 128 == 0. */
int dwm_fp8_block_requant(const uint8_t *w, const float *scale, int64_t K, int64_t N, int input_nk,
                          uint8_t *w_out, float *scale_out, int32_t *status, void *stream);

/* ---------------------------------------------------------------------- */
/* Router (the producer of topk_ids / topk_weights).                       */
/* ---------------------------------------------------------------------- */

/* Top-k routing "exactly as fused_moe_func" (_fused_moe_fp4_routing,
 * patches/tpu-inference-experimental/fused-moe-fp4/0901-...:656-687):
 * scores = score_fn(logits) in f32; experts = hash_ids when given, else the
 * top k of scores + bias when bias is given, else of scores (larger first,
 * ties to the lower expert id, as lax.top_k); weights = the experts'
 * (unbiased) scores; renormalize divides by their sum over k in order;
 * tokens t >= *num_valid_tokens get expert 0 and weight 0; weights are cast
 * to weights_dtype (bf16 round to nearest even, or f32).
 *   logits: [T, E] bf16 or f32; bias: f32 [E] or NULL; hash_ids: int32
 *   [T, topk] or NULL; num_valid_tokens: device int32[1] or NULL (all valid).
 *   weights_out: [T, topk]; ids_out: int32 [T, topk].
 * Requires E <= 1024, topk <= min(E, 64). */
int dwm_route_topk(const void *logits, int logits_dtype, int64_t T, int64_t E, int topk, int score_fn,
                   const float *bias, const int32_t *hash_ids, int renormalize,
                   const int32_t *num_valid_tokens, void *weights_out, int weights_dtype, int32_t *ids_out,
                   void *stream);

/* dedupe_topk (0901-...:98-121): for j = 1 .. topk-1 a repeat of an earlier
 * expert id adds its weight (f32) to the first occurrence and is re-pointed
 * at the first id in [0, min(2 topk, E)) no column of the token holds (0
 * when all are held), with weight 0.  w: f32 [T, topk]; ids: int32
 * [T, topk].  Requires topk <= 64. */
int dwm_dedupe_topk(const float *w_in, const int32_t *ids_in, int64_t T, int topk, int64_t E, float *w_out,
                    int32_t *ids_out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* DWTPU_MOE_H_ */
