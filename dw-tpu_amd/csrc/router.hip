// MoE router: scores -> top-k -> renormalize -> invalid-token mask -> cast
// (the routing "exactly as fused_moe_func" restated in
// patches/tpu-inference-experimental/fused-moe-fp4/0901-...:656-687), and
// dedupe_topk (0901-...:98-121), which makes a token's expert ids distinct.
//
// One wavefront per token: lane l holds experts l, l + 64, ... (coalesced
// loads of the logits row), the scores are computed in registers, and the
// top-k runs as k wave-wide arg-max rounds (larger key first, then the lower
// expert id, as lax.top_k orders ties).  Lane j keeps result j, so the
// outputs are written by lanes 0 .. k-1 without a staging buffer.
#include "common.h"

namespace dwm {

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
  return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

// Key order of the selection: a before b when a's key is larger, or equal
// with a lower expert id.  Taken experts carry taken = true and lose to all.
__device__ __forceinline__ bool key_before(float ka, int ea, bool ta, float kb, int eb, bool tb) {
  if (ta != tb) return tb;
  if (ka != kb) return ka > kb;
  return ea < eb;
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
  float p[VPL], key[VPL];
  bool taken[VPL];
  float x[VPL];
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + 64 * i;
    float v = -__builtin_inff();
    if (e < E) {
      v = logits_bf16 ? bf16_bits_to_f32(((const uint16_t *)logits)[t * E + e])
                      : ((const float *)logits)[t * E + e];
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
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + 64 * i;
    key[i] = (bias != nullptr && e < E) ? p[i] + bias[e] : p[i];
    taken[i] = e >= E;
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
      v = __shfl(v, id & 63, 64);
      if (lane == j) {
        my_w = v;
        my_id = id;
      }
    }
  } else {
    for (int j = 0; j < topk; ++j) {
      float bk = 0.0f, bw = 0.0f;
      int be = 0x7FFFFFFF;
      bool bt = true;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int e = lane + 64 * i;
        if (key_before(key[i], e, taken[i], bk, be, bt)) {
          bk = key[i];
          be = e;
          bt = taken[i];
          bw = p[i];
        }
      }
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) {
        const float ok = __shfl_xor(bk, d, 64), ow = __shfl_xor(bw, d, 64);
        const int oe = __shfl_xor(be, d, 64);
        const bool ot = __shfl_xor((int)bt, d, 64) != 0;
        if (key_before(ok, oe, ot, bk, be, bt)) {
          bk = ok;
          be = oe;
          bt = ot;
          bw = ow;
        }
      }
      // Every lane now holds the winner; its owner marks it taken.
#pragma unroll
      for (int i = 0; i < VPL; ++i)
        if (lane + 64 * i == be) taken[i] = true;
      if (lane == j) {
        my_w = bw;
        my_id = be;
      }
    }
  }
  if (renorm) {
    float tot = 0.0f;  // the sum over k in order
    for (int j = 0; j < topk; ++j) tot += __shfl(my_w, j, 64);
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
