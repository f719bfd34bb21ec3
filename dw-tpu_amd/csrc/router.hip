// MoE router: scores -> top-k -> renormalize -> invalid-token mask -> cast
// (the routing "exactly as fused_moe_func" restated in
// patches/tpu-inference-experimental/fused-moe-fp4/0901-...:656-687), and
// dedupe_topk (0901-...:98-121), which makes a token's expert ids distinct.
//
// One wavefront per token: lane l holds experts l, l + 64, ... (coalesced
// loads of the logits row), the scores are computed in registers, and the
// top-k runs as k wave-wide arg-max rounds (larger key first, then the lower
// expert id, as lax.top_k orders ties): a 32-bit max of the keys, then a
// ballot per slot for the lowest id holding it.
// Lane j keeps result j, so the outputs are written by lanes 0 .. k-1
// without a staging buffer.
#include "common.h"

namespace dwm {

// Wave-wide reductions without LDS traffic: four DPP steps combine the 16
// lanes of each row (pairs, quads, the two halves of 8, the two halves of
// 16, every lane ending with its row's result), then the four rows are read
// as scalars and combined in row order.  The result is wave-uniform.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}

template <class F>
__device__ __forceinline__ float wave_reduce_f32(float v, F op) {
  v = op(v, __builtin_bit_cast(float, dpp_u32<kDppXor1>(__builtin_bit_cast(uint32_t, v))));
  v = op(v, __builtin_bit_cast(float, dpp_u32<kDppXor2>(__builtin_bit_cast(uint32_t, v))));
  v = op(v, __builtin_bit_cast(float, dpp_u32<kDppHalfMirror>(__builtin_bit_cast(uint32_t, v))));
  v = op(v, __builtin_bit_cast(float, dpp_u32<kDppMirror>(__builtin_bit_cast(uint32_t, v))));
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  float r = __builtin_bit_cast(float, lane_u32(b, 0));
  r = op(r, __builtin_bit_cast(float, lane_u32(b, 16)));
  r = op(r, __builtin_bit_cast(float, lane_u32(b, 32)));
  return op(r, __builtin_bit_cast(float, lane_u32(b, 48)));
}

__device__ __forceinline__ float wave_max_f32(float v) {
  return wave_reduce_f32(v, [](float a, float b) { return fmaxf(a, b); });
}

__device__ __forceinline__ float wave_sum_f32(float v) {
  return wave_reduce_f32(v, [](float a, float b) { return a + b; });
}

// Selection order: a larger key first, then the lower expert id (lax.top_k's
// tie order).  A candidate's key is its score's bits made monotone as an
// unsigned integer (flip all bits of a negative, set the sign bit of a
// non-negative); -0 is folded into +0 first, as the float comparison treats
// them as equal.  Every number then maps to at least 0x007FFFFF (-inf), a
// NaN to 1 (below every number; NaNs tie by id), and a taken expert or a
// lane past E holds 0 and loses to every candidate.
__device__ __forceinline__ uint32_t select_key(float key) {
  uint32_t b = __builtin_bit_cast(uint32_t, key == 0.0f ? 0.0f : key);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return key != key ? 1u : b;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<kDppXor1>(v));
  v = max(v, dpp_u32<kDppXor2>(v));
  v = max(v, dpp_u32<kDppHalfMirror>(v));
  v = max(v, dpp_u32<kDppMirror>(v));
  return max(max(lane_u32(v, 0), lane_u32(v, 16)), max(lane_u32(v, 32), lane_u32(v, 48)));
}

template <int VPL>
__global__ __launch_bounds__(256) void route_topk_kernel(const void *__restrict__ logits, int logits_bf16, int64_t T,
                                                         int E, int topk, int score_fn,
                                                         const float *__restrict__ bias,
                                                         const int32_t *__restrict__ hash_ids, int renorm,
                                                         const int32_t *__restrict__ num_valid,
                                                         void *__restrict__ w_out, int w_bf16,
                                                         int32_t *__restrict__ ids_out) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float p[VPL];
  float x[VPL];
  float bv[VPL];  // the correction bias, loaded with the logits (one memory round trip)
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + 64 * i;
    float v = -__builtin_inff();
    bv[i] = 0.0f;
    if (e < E) {
      v = logits_bf16 ? bf16_bits_to_f32(((const uint16_t *)logits)[t * E + e])
                      : ((const float *)logits)[t * E + e];
      if (bias != nullptr) bv[i] = bias[e];
    }
    x[i] = v;
    m = fmaxf(m, v);
  }
  if (score_fn == DWM_SCORE_SOFTMAX) {
    m = wave_max_f32(m);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      x[i] = lane + 64 * i < E ? expf(x[i] - m) : 0.0f;
      s += x[i];
    }
    s = wave_sum_f32(s);
#pragma unroll
    for (int i = 0; i < VPL; ++i) p[i] = x[i] / s;
  } else if (score_fn == DWM_SCORE_SIGMOID) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) p[i] = 1.0f / (1.0f + expf(-x[i]));
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i) p[i] = sqrtf(fmaxf(x[i], 0.0f) + log1pf(expf(-fabsf(x[i]))));
  }
  uint32_t cand[VPL];  // selection key of expert lane + 64 i; 0 once taken (or past E)
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + 64 * i;
    cand[i] = e < E ? select_key(bias != nullptr ? p[i] + bv[i] : p[i]) : 0u;
  }
  float my_w = 0.0f;  // result j = lane
  int my_id = 0;
  if (hash_ids != nullptr) {
    for (int j = 0; j < topk; ++j) {
      const int id = hash_ids[t * topk + j];  // uniform across the wave
      const int slot = id >> 6;
      float v = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) v = slot == i ? p[i] : v;
      v = __builtin_bit_cast(float, lane_u32(__builtin_bit_cast(uint32_t, v), id & 63));
      if (lane == j) {
        my_w = v;
        my_id = id;
      }
    }
  } else {
    for (int j = 0; j < topk; ++j) {
      // The largest key (wave-uniform), then its lowest expert id: experts
      // of slot i are lane + 64 i, so the first slot holding it wins, and
      // in that slot the lowest lane.  topk <= E, so a candidate is left.
      uint32_t best = cand[0];
#pragma unroll
      for (int i = 1; i < VPL; ++i) best = max(best, cand[i]);
      best = wave_max_u32(best);
      int slot = 0;
      uint64_t hit = 0;
#pragma unroll
      for (int i = VPL - 1; i >= 0; --i) {
        const uint64_t b = __ballot(cand[i] == best);
        if (b != 0) {
          slot = i;
          hit = b;
        }
      }
      const int owner = __ffsll((long long)hit) - 1;
      const int id = owner + 64 * slot;
      // The owner marks it taken and hands over its unbiased weight.
      float v = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) v = slot == i ? p[i] : v;
      v = __builtin_bit_cast(float, lane_u32(__builtin_bit_cast(uint32_t, v), owner));
      if (lane == owner) {
#pragma unroll
        for (int i = 0; i < VPL; ++i) cand[i] = slot == i ? 0u : cand[i];
      }
      if (lane == j) {
        my_w = v;
        my_id = id;
      }
    }
  }
  if (renorm) {
    float tot = 0.0f;  // the sum over k in order
    for (int j = 0; j < topk; ++j) tot += __builtin_bit_cast(float, lane_u32(__builtin_bit_cast(uint32_t, my_w), j));
    my_w = my_w / tot;
  }
  if (num_valid != nullptr && t >= (int64_t)num_valid[0]) {
    my_w = 0.0f;
    my_id = 0;
  }
  if (lane < topk) {
    if (w_bf16) ((uint16_t *)w_out)[t * topk + lane] = f32_to_bf16_bits(my_w);
    else ((float *)w_out)[t * topk + lane] = my_w;
    ids_out[t * topk + lane] = my_id;
  }
}

// dedupe_topk: one wavefront per token, lane j = column j.
__global__ __launch_bounds__(256) void dedupe_topk_kernel(const float *__restrict__ w_in,
                                                          const int32_t *__restrict__ ids_in, int64_t T, int topk,
                                                          int64_t E, float *__restrict__ w_out,
                                                          int32_t *__restrict__ ids_out) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const bool col = lane < topk;
  float w = col ? w_in[t * topk + lane] : 0.0f;
  int id = col ? ids_in[t * topk + lane] : -1;
  const int ncand = (int)min((int64_t)2 * topk, E);
  for (int j = 1; j < topk; ++j) {
    const int idj = __shfl(id, j, 64);
    const float wj = __shfl(w, j, 64);
    const uint64_t same = __ballot(lane < j && id == idj);
    const bool dup = same != 0;
    const int first = dup ? __ffsll((long long)same) - 1 : 0;
    // The reference's scatter-add runs for every token (adding +0.0 when
    // there is no repeat).
    if (lane == first) w = w + (dup ? wj : 0.0f);
    // Candidates 0 .. ncand-1 (lane c) held by any column of the token now.
    // Every lane runs every shuffle: a shuffle reads 0 from a lane that is
    // not active, so it must not sit behind a per-lane condition.
    bool used = false;
    for (int q = 0; q < topk; ++q) {
      const int idq = __shfl(id, q, 64);
      used |= idq == lane;
    }
    const uint64_t freem = __ballot(lane < ncand && !used);
    const int fr = freem != 0 ? __ffsll((long long)freem) - 1 : 0;
    if (lane == j && dup) {
      id = fr;
      w = 0.0f;
    }
  }
  if (col) {
    w_out[t * topk + lane] = w;
    ids_out[t * topk + lane] = id;
  }
}

}  // namespace dwm

using namespace dwm;

extern "C" int dwm_route_topk(const void *logits, int logits_dtype, int64_t T, int64_t E, int topk, int score_fn,
                              const float *bias, const int32_t *hash_ids, int renormalize,
                              const int32_t *num_valid_tokens, void *weights_out, int weights_dtype,
                              int32_t *ids_out, void *stream) {
  clear_error();
  DWM_CHECK_ARG(T >= 0 && E > 0, "route_topk: bad sizes T=%lld E=%lld", (long long)T, (long long)E);
  DWM_CHECK_ARG(logits_dtype == DWM_BF16 || logits_dtype == DWM_F32, "route_topk: bad logits dtype %d",
                logits_dtype);
  DWM_CHECK_ARG(weights_dtype == DWM_BF16 || weights_dtype == DWM_F32, "route_topk: bad weights dtype %d",
                weights_dtype);
  DWM_CHECK_ARG(score_fn == DWM_SCORE_SOFTMAX || score_fn == DWM_SCORE_SIGMOID ||
                    score_fn == DWM_SCORE_SQRTSOFTPLUS,
                "route_topk: bad score_fn %d", score_fn);
  DWM_CHECK_ARG(topk >= 1 && topk <= E, "route_topk: need 1 <= topk <= E (topk=%d E=%lld)", topk, (long long)E);
  DWM_UNSUPPORTED_IF(E > 1024 || topk > 64, "route_topk: E <= 1024 and topk <= 64 supported (E=%lld topk=%d)",
                     (long long)E, topk);
  DWM_UNSUPPORTED_IF(T > (int64_t)4 * 0x7FFFFFFF, "route_topk: too many tokens");
  if (T == 0) return DWM_OK;
  DWM_CHECK_ARG(logits && weights_out && ids_out, "route_topk: null pointer");
  hipStream_t st = as_stream(stream);
  const dim3 grid((unsigned)((T + 3) / 4)), block(256);
  const int lb = logits_dtype == DWM_BF16, wb = weights_dtype == DWM_BF16;
#define ROUTE(V)                                                                                                  \
  hipLaunchKernelGGL(route_topk_kernel<V>, grid, block, 0, st, logits, lb, T, (int)E, topk, score_fn, bias,     \
                     hash_ids, renormalize ? 1 : 0, num_valid_tokens, weights_out, wb, ids_out)
  if (E <= 64) ROUTE(1);
  else if (E <= 128) ROUTE(2);
  else if (E <= 256) ROUTE(4);
  else if (E <= 512) ROUTE(8);
  else ROUTE(16);
#undef ROUTE
  return launch_status("route_topk");
}

extern "C" int dwm_dedupe_topk(const float *w_in, const int32_t *ids_in, int64_t T, int topk, int64_t E,
                               float *w_out, int32_t *ids_out, void *stream) {
  clear_error();
  DWM_CHECK_ARG(T >= 0 && E > 0 && topk >= 1, "dedupe_topk: bad sizes T=%lld topk=%d E=%lld", (long long)T, topk,
                (long long)E);
  DWM_UNSUPPORTED_IF(topk > 64, "dedupe_topk: topk <= 64 supported (topk=%d)", topk);
  DWM_UNSUPPORTED_IF(T > (int64_t)4 * 0x7FFFFFFF, "dedupe_topk: too many tokens");
  if (T == 0) return DWM_OK;
  DWM_CHECK_ARG(w_in && ids_in && w_out && ids_out, "dedupe_topk: null pointer");
  hipLaunchKernelGGL(dedupe_topk_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, as_stream(stream), w_in,
                     ids_in, T, topk, E, w_out, ids_out);
  return launch_status("dedupe_topk");
}
