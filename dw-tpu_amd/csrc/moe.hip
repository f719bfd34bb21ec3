// MoE dispatch (expert-stable counting sort), row gather and combine.
//
// Dispatch replaces jnp.argsort(topk_ids.flatten()) + argsort // topk +
// one_hot(...).sum(0) (patches/tpu-inference-ext/0405-moe-fast-dispatch.patch:70-98,
// kernels/tpu_inference/layers/common/moe_fast_dispatch.py:41-44) with a
// counting sort that is bit-exact to a stable argsort, in three launches
// (one block for batches of up to 8192 ids, dispatch_fused_kernel):
//   1. per 1024-id chunk, an LDS histogram -> counts[chunk][expert]
//   2. one block: group sizes, exclusive offsets, per-(chunk, expert) bases
//   3. per chunk, in id order (256 ids per step, wave by wave): each lane's
//      rank among equal ids of its wave comes from ballots over the id bits;
//      earlier waves' counts come from LDS.  Position = base + rank.
// Ids outside [0, E) get the key E, i.e. they sort after every valid id.
//
// This file is compiled with -ffp-contract=off: the combine's f32 products
// and sums must stay separately rounded (moe_fast_combine.py:44-54).
#include <mutex>

#include "common.h"

namespace dwm {

constexpr int kChunk = 1024;
constexpr int kDispThreads = 256;
constexpr int kMaxExperts = 1024;

__device__ __forceinline__ int dispatch_key(int32_t id, int E, bool *bad) {
  if (id < 0 || id >= E) {
    *bad = true;
    return E;
  }
  return id;
}

__global__ __launch_bounds__(kDispThreads) void dispatch_count_kernel(const int32_t *ids, int64_t n,
                                                                      int E, int32_t *counts,
                                                                      int32_t *flags) {
  __shared__ int s_hist[kMaxExperts + 1];
  for (int e = threadIdx.x; e <= E; e += kDispThreads) s_hist[e] = 0;
  __syncthreads();
  bool bad = false;
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  for (int i = 0; i < kChunk / kDispThreads; ++i) {
    const int64_t j = base + i * kDispThreads + threadIdx.x;
    if (j < n) atomicAdd(&s_hist[dispatch_key(ids[j], E, &bad)], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += kDispThreads)
    counts[(int64_t)blockIdx.x * (E + 1) + e] = s_hist[e];
  if (bad && flags) atomicOr(flags, 1);
}

// One block.  counts[c][e] -> base position of chunk c's first id of key e.
__global__ __launch_bounds__(1024) void dispatch_scan_kernel(int32_t *counts, int nchunks, int E,
                                                             int32_t *group_sizes,
                                                             int32_t *group_offsets) {
  __shared__ int s_tot[kMaxExperts + 1];
  __shared__ int s_off[kMaxExperts + 1];
  __shared__ int s_part[1024];  // [G][E + 1] sums of each chunk run
  // counts[nchunks][E + 1]: thread (g, e) owns column e of the contiguous
  // chunk run g, G = blockDim / (E + 1) runs (loads coalesced along e).  With
  // more columns than threads (G = 0) each thread walks whole columns.
  const int C = E + 1;
  const int G = (int)blockDim.x / C;
  const int tid = threadIdx.x;
  const int L = G > 0 ? (nchunks + G - 1) / G : 0;
  const int e = G > 0 ? tid % C : 0, g = G > 0 ? tid / C : 0;
  const bool own = G > 0 && g < G;
  const int c_lo = own ? min(nchunks, g * L) : 0, c_hi = own ? min(nchunks, c_lo + L) : 0;
  if (own) {
    int sum = 0;
    for (int c = c_lo; c < c_hi; ++c) sum += counts[(int64_t)c * C + e];
    s_part[g * C + e] = sum;
  }
  __syncthreads();
  for (int ee = tid; ee < C; ee += blockDim.x) {
    int t = 0;
    if (G > 0)
      for (int gg = 0; gg < G; ++gg) t += s_part[gg * C + ee];
    else
      for (int c = 0; c < nchunks; ++c) t += counts[(int64_t)c * C + ee];
    s_tot[ee] = t;
  }
  __syncthreads();
  if (tid < 64) {
    const int lane = tid;
    int carry = 0;
    for (int b = 0; b < C; b += 64) {
      const int ee = b + lane;
      const int v = ee < C ? s_tot[ee] : 0;
      const int inc = wave_inclusive_scan(v);
      if (ee < C) s_off[ee] = carry + inc - v;
      carry += wave_last(inc);
    }
  }
  __syncthreads();
  for (int ee = tid; ee < C; ee += blockDim.x) {
    if (ee < E) group_sizes[ee] = s_tot[ee];
    if (group_offsets) group_offsets[ee] = s_off[ee];  // entry E = number of valid ids
    if (G == 0) {
      int run = s_off[ee];
      for (int c = 0; c < nchunks; ++c) {
        const int64_t idx = (int64_t)c * C + ee;
        const int v = counts[idx];
        counts[idx] = run;
        run += v;
      }
    }
  }
  if (own) {
    int run = s_off[e];
    for (int gg = 0; gg < g; ++gg) run += s_part[gg * C + e];
    for (int c = c_lo; c < c_hi; ++c) {
      const int64_t idx = (int64_t)c * C + e;
      const int v = counts[idx];
      counts[idx] = run;
      run += v;
    }
  }
}

__global__ __launch_bounds__(kDispThreads) void dispatch_scatter_kernel(
    const int32_t *ids, int64_t n, int topk, int E, const int32_t *bases, int32_t *perm,
    int32_t *tok_sorted, int32_t *revert) {
  __shared__ int s_run[kMaxExperts + 1];
  __shared__ int s_wcnt[kDispThreads / 64][kMaxExperts + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e <= E; e += kDispThreads) {
    s_run[e] = bases[(int64_t)blockIdx.x * (E + 1) + e];
#pragma unroll
    for (int w = 0; w < kDispThreads / 64; ++w) s_wcnt[w][e] = 0;
  }
  int nbits = 0;
  while ((1 << nbits) <= E) ++nbits;  // keys 0..E
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  for (int i = 0; i < kChunk / kDispThreads; ++i) {
    const int64_t j = base + i * kDispThreads + tid;
    const bool active = j < n;
    bool bad = false;
    const int key = active ? dispatch_key(ids[j], E, &bad) : 0;
    uint64_t peers = __ballot(active);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (key >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int rank = __popcll(peers & ((1ull << lane) - 1ull));
    const int cnt = __popcll(peers);
    const bool leader = active && rank == 0;
    if (leader) s_wcnt[wave][key] = cnt;
    __syncthreads();
    if (active) {
      int pos = s_run[key] + rank;
      for (int w = 0; w < wave; ++w) pos += s_wcnt[w][key];
      perm[pos] = (int32_t)j;
      tok_sorted[pos] = (int32_t)(j / topk);
      revert[j] = pos;
    }
    __syncthreads();
    if (leader) {
      atomicAdd(&s_run[key], cnt);
      s_wcnt[wave][key] = 0;
    }
    __syncthreads();
  }
}

// Small batches (n <= kFusedMax ids) over 64 or more experts (fewer take
// dispatch_small_kernel below): one block of 1024 threads runs all three
// steps -- the LDS histogram, the scan (wave 0) and the stable scatter in
// 1024-id steps -- in one launch, with no workspace round trip.
constexpr int kFusedThreads = 1024, kFusedMax = 8192;

__global__ __launch_bounds__(kFusedThreads) void dispatch_fused_kernel(const int32_t *ids, int64_t n, int topk,
                                                                       int E, int32_t *perm, int32_t *tok_sorted,
                                                                       int32_t *revert, int32_t *group_sizes,
                                                                       int32_t *group_offsets, int32_t *flags) {
  constexpr int W = kFusedThreads / 64;
  __shared__ int s_run[kMaxExperts + 1];     // counts, then the next position of each key
  __shared__ int s_wcnt[W][kMaxExperts + 1];  // this step's count of each key per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e <= E; e += kFusedThreads) {
    s_run[e] = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) s_wcnt[w][e] = 0;
  }
  __syncthreads();
  bool bad = false;
  for (int64_t j = tid; j < n; j += kFusedThreads) atomicAdd(&s_run[dispatch_key(ids[j], E, &bad)], 1);
  if (bad && flags) atomicOr(flags, 1);
  __syncthreads();
  if (wave == 0) {
    int carry = 0;
    for (int b = 0; b <= E; b += 64) {
      const int e = b + lane;
      const int v = e <= E ? s_run[e] : 0;
      const int inc = wave_inclusive_scan(v);
      if (e <= E) {
        if (e < E) group_sizes[e] = v;
        if (group_offsets) group_offsets[e] = carry + inc - v;  // entry E = number of valid ids
        s_run[e] = carry + inc - v;
      }
      carry += wave_last(inc);
    }
  }
  int nbits = 0;
  while ((1 << nbits) <= E) ++nbits;  // keys 0..E
  __syncthreads();
  for (int64_t base = 0; base < n; base += kFusedThreads) {
    const int64_t j = base + tid;
    const bool active = j < n;
    bool b2 = false;
    const int key = active ? dispatch_key(ids[j], E, &b2) : 0;
    uint64_t peers = __ballot(active);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (key >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int rank = __popcll(peers & ((1ull << lane) - 1ull));
    const int cnt = __popcll(peers);
    const bool leader = active && rank == 0;
    if (leader) s_wcnt[wave][key] = cnt;
    __syncthreads();
    if (active) {
      int pos = s_run[key] + rank;
      for (int w = 0; w < wave; ++w) pos += s_wcnt[w][key];
      perm[pos] = (int32_t)j;
      tok_sorted[pos] = (int32_t)(j / topk);
      revert[j] = pos;
    }
    __syncthreads();
    if (leader) {
      atomicAdd(&s_run[key], cnt);
      s_wcnt[wave][key] = 0;
    }
    __syncthreads();
  }
}


// Small batches over few experts (n <= kFusedMax ids, E + 1 <= 64 keys):
// the scattered stores, not the ranking, set the time of a one-block
// dispatch, so the ids are split into portions of 512 over up to 16 blocks.
// Every block counts all n ids (cheap: 16 waves, one 64-id round each per
// 1024 ids) by key -- in total and before its portion -- and ranks its own
// portion; lane e of a wave counts key e from the key bits' ballots, and a
// lane's rank within a round is the lanes below it holding its key.  An id
// lands at key offset + ids of its key before the portion + before its round
// in the portion + its rank in the round: the stable order of j.  Block 0
// writes the group sizes and offsets.  No atomics and two block barriers.
constexpr int kSmallMaxKeys = 64, kSmallPortion = 512;

__global__ __launch_bounds__(kFusedThreads) void dispatch_small_kernel(const int32_t *ids, int64_t n, int topk,
                                                                       int E, int32_t *perm, int32_t *tok_sorted,
                                                                       int32_t *revert, int32_t *group_sizes,
                                                                       int32_t *group_offsets, int32_t *flags) {
  constexpr int W = kFusedThreads / 64, PR = kSmallPortion / 64;     // waves; rounds per portion
  constexpr int RMAX = kFusedMax / kFusedThreads;                      // rounds per wave
  static_assert(PR <= W, "a portion's rounds fall on distinct waves");
  __shared__ int s_tot[W][kSmallMaxKeys], s_bef[W][kSmallMaxKeys];
  __shared__ int s_rc[PR][kSmallMaxKeys];  // per round of the portion: count of each key
  __shared__ int s_base[kSmallMaxKeys], s_rp[PR][kSmallMaxKeys];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int NR = (int)((n + 63) >> 6);  // 64-id rounds
  const int r0 = blockIdx.x * PR;       // the portion's first round
  int nbits = 0;
  while ((1 << nbits) <= E) ++nbits;  // keys 0 .. E
  const uint64_t lt = (1ull << lane) - 1ull;
  // Round wave + W i; every round's id is loaded before the first is counted.
  int key[RMAX];
#pragma unroll
  for (int i = 0; i < RMAX; ++i) {
    const int64_t j = (int64_t)(wave + W * i) * 64 + lane;
    key[i] = j < n ? ids[j] : 0;
  }
  int tot = 0, bef = 0, myrank = 0, mykey = 0, myq = -1;  // lane e: key e's counts
  bool bad = false;
#pragma unroll
  for (int i = 0; i < RMAX; ++i) {
    const int r = wave + W * i;
    if (r < NR) {
      const int64_t j = (int64_t)r * 64 + lane;
      const bool active = j < n;
      const int k = active ? dispatch_key(key[i], E, &bad) : 0;
      uint64_t peers = __ballot(active), mine = peers;  // lanes holding my key; holding key `lane`
      for (int b = 0; b < nbits; ++b) {
        const uint64_t m = __ballot(active && ((k >> b) & 1));
        peers &= ((k >> b) & 1) ? m : ~m;
        mine &= ((lane >> b) & 1) ? m : ~m;
      }
      const int c = lane <= E ? __popcll(mine) : 0;
      tot += c;
      if (r < r0) bef += c;
      const int q = r - r0;
      if (q >= 0 && q < PR) {  // a round of this block's portion (one per wave)
        if (lane <= E) s_rc[q][lane] = c;
        myq = q;
        mykey = k;
        myrank = __popcll(peers & lt);
      }
    }
  }
  if (lane <= E) {
    s_tot[wave][lane] = tot;
    s_bef[wave][lane] = bef;
  }
  if (bad && flags) atomicOr(flags, 1);
  __syncthreads();
  if (wave == 0) {
    int t = 0, bf = 0;
    for (int w = 0; w < W; ++w) {
      t += lane <= E ? s_tot[w][lane] : 0;
      bf += lane <= E ? s_bef[w][lane] : 0;
    }
    const int off = wave_inclusive_scan(t) - t;
    if (lane <= E) {
      if (blockIdx.x == 0) {
        if (lane < E) group_sizes[lane] = t;
        if (group_offsets) group_offsets[lane] = off;  // entry E = number of valid ids
      }
      s_base[lane] = off + bf;
      int run = 0;  // ids of key `lane` in the portion's rounds before q
      for (int q = 0; q < PR; ++q) {
        s_rp[q][lane] = run;
        run += r0 + q < NR ? s_rc[q][lane] : 0;
      }
    }
  }
  __syncthreads();
  if (myq >= 0) {
    const int64_t j = (int64_t)(r0 + myq) * 64 + lane;
    if (j < n) {
      const int p = s_base[mykey] + s_rp[myq][mykey] + myrank;
      perm[p] = (int32_t)j;
      tok_sorted[p] = (int32_t)(j / topk);
      revert[j] = p;
    }
  }
}

// Floor division by a positive divisor (Python / JAX `//` on integers).
__device__ __forceinline__ int64_t floor_div(int64_t i, int64_t d) {
  return i >= 0 ? i / d : -((-i + d - 1) / d);
}

// out[r] = src[idx[r] // div] (div = 1: a plain row gather; div = topk: the
// dispatch gather of the token rows behind an expert-sorted argsort).
template <typename V>
__global__ __launch_bounds__(256) void row_gather_kernel(const char *src, int64_t src_rows,
                                                         int64_t row_bytes, const int32_t *idx,
                                                         int64_t rows, char *out, int div) {
  const int64_t nv = row_bytes / (int64_t)sizeof(V);
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const int64_t s = gather_index(div == 1 ? (int64_t)idx[r] : floor_div(idx[r], div), src_rows);
    const V *sp = (const V *)(src + s * row_bytes);
    V *dp = (V *)(out + r * row_bytes);
    for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) __builtin_nontemporal_store(sp[i], dp + i);
  }
}

__device__ __forceinline__ float load_f32(const void *p, int dtype, int64_t i) {
  return dtype == DWM_F32 ? ((const float *)p)[i]
                          : bf16_bits_to_f32(((const uint16_t *)p)[i]);
}

// Block (column chunk, token): each thread owns 8 consecutive columns of one
// token.  The token's top-k rows are read in groups of KG, all loads of a
// group issued before the group is summed (in k order, so the result is the
// same left-to-right f32 sum), and the 8 outputs leave in 16-byte stores.
constexpr int kCombineKG = 8;

template <int XF32>
__device__ __forceinline__ void load8_f32(const void *x, int64_t o, bool full, int64_t H, int64_t c, float *v) {
  if (full && !XF32) {
    const u32x4_t q = *(const u32x4_t *)((const uint16_t *)x + o);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __builtin_bit_cast(float, q[i] << 16);
      v[2 * i + 1] = __builtin_bit_cast(float, q[i] & 0xFFFF0000u);
    }
  } else if (full) {
    const f32x4_t q0 = *(const f32x4_t *)((const float *)x + o);
    const f32x4_t q1 = *(const f32x4_t *)((const float *)x + o + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = q0[i];
      v[4 + i] = q1[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = c + i < H ? load_f32(x, XF32 ? DWM_F32 : DWM_BF16, o + i) : 0.0f;
  }
}

template <int XF32, int OF32>
__global__ __launch_bounds__(256) void combine_kernel(const void *x, int64_t x_rows, int64_t H,
                                                      const int32_t *idx, const void *w, int w_dtype,
                                                      int64_t T, int topk, void *out, int vec) {
  const int64_t c = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (c >= H) return;
  const bool full = vec && c + 8 <= H;
  for (int64_t t = blockIdx.y; t < T; t += gridDim.y) {
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    for (int k0 = 0; k0 < topk; k0 += kCombineKG) {
      float v[kCombineKG][8], wk[kCombineKG];
#pragma unroll
      for (int g = 0; g < kCombineKG; ++g) {
        if (k0 + g < topk) {
          const int64_t r = gather_index(idx[t * topk + k0 + g], x_rows);
          wk[g] = load_f32(w, w_dtype, t * topk + k0 + g);
          load8_f32<XF32>(x, r * H + c, full, H, c, v[g]);
        }
      }
#pragma unroll
      for (int g = 0; g < kCombineKG; ++g) {
        if (k0 + g < topk) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float p = v[g][i] * wk[g];  // separately rounded product
            acc[i] = acc[i] + p;              // then sum, k ascending from +0.0
          }
        }
      }
    }
    if (full) {
      if (OF32) {
        *(f32x4_t *)((float *)out + t * H + c) = f32x4_t{acc[0], acc[1], acc[2], acc[3]};
        *(f32x4_t *)((float *)out + t * H + c + 4) = f32x4_t{acc[4], acc[5], acc[6], acc[7]};
      } else {
        u32x4_t q;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          q[i] = f32x2_to_bf16x2_bits(acc[2 * i], acc[2 * i + 1]);
        *(u32x4_t *)((uint16_t *)out + t * H + c) = q;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (c + i >= H) break;
        if (OF32) ((float *)out)[t * H + c + i] = acc[i];
        else ((uint16_t *)out)[t * H + c + i] = f32_to_bf16_bits(acc[i]);
      }
    }
  }
}

// The combine for bf16 rows with 16-byte aligned rows (H % 8 == 0): the
// same arithmetic as combine_kernel, but each row's 8 values stay packed
// (one 16-byte register quad per row, widened while accumulating), so a
// thread holds its kCombineKG rows in 32 registers and every block of the
// decode shapes is resident at once (8 waves per SIMD).
template <int OF32>
__global__ __launch_bounds__(256) void combine_bf16_kernel(const uint16_t *__restrict__ x, int64_t x_rows, int64_t H,
                                                           const int32_t *__restrict__ idx, const void *w,
                                                           int w_dtype, int64_t T, int topk, void *out) {
  const int64_t c = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (c >= H) return;
  for (int64_t t = blockIdx.y; t < T; t += gridDim.y) {
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    for (int k0 = 0; k0 < topk; k0 += kCombineKG) {
      u32x4_t raw[kCombineKG];
      float wk[kCombineKG];
#pragma unroll
      for (int g = 0; g < kCombineKG; ++g) {
        if (k0 + g < topk) {
          const int64_t r = gather_index(idx[t * topk + k0 + g], x_rows);
          wk[g] = load_f32(w, w_dtype, t * topk + k0 + g);
          raw[g] = *(const u32x4_t *)(x + r * H + c);
        }
      }
#pragma unroll
      for (int g = 0; g < kCombineKG; ++g) {
        if (k0 + g < topk) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float lo = __builtin_bit_cast(float, raw[g][i] << 16);
            const float hi = __builtin_bit_cast(float, raw[g][i] & 0xFFFF0000u);
            acc[2 * i] = acc[2 * i] + lo * wk[g];          // separately rounded product,
            acc[2 * i + 1] = acc[2 * i + 1] + hi * wk[g];  // then sum, k ascending from +0.0
          }
        }
      }
    }
    if (OF32) {
      *(f32x4_t *)((float *)out + t * H + c) = f32x4_t{acc[0], acc[1], acc[2], acc[3]};
      *(f32x4_t *)((float *)out + t * H + c + 4) = f32x4_t{acc[4], acc[5], acc[6], acc[7]};
    } else {
      u32x4_t q;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        q[i] = f32x2_to_bf16x2_bits(acc[2 * i], acc[2 * i + 1]);
      *(u32x4_t *)((uint16_t *)out + t * H + c) = q;
    }
  }
}

// The dispatch launches for n = T * topk ids with chunk counters `counts`
// (nchunks * (E + 1) int32, fully written by the count kernel before they are
// read, so they need no clearing).
static int dispatch_launch(const int32_t *topk_ids, int64_t n, int topk, int num_experts, int32_t *perm,
                           int32_t *tok_sorted, int32_t *revert, int32_t *group_sizes, int32_t *group_offsets,
                           int32_t *flags, int32_t *counts, hipStream_t st) {
  const int64_t nchunks = (n + kChunk - 1) / kChunk;
  if (n == 0) {
    hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(1024), 0, st, counts, 0, num_experts,
                       group_sizes, group_offsets);
    return launch_status("moe_dispatch");
  }
  if (n <= kFusedMax && num_experts < kSmallMaxKeys) {
    const unsigned blocks = (unsigned)((n + kSmallPortion - 1) / kSmallPortion);
    hipLaunchKernelGGL(dispatch_small_kernel, dim3(blocks), dim3(kFusedThreads), 0, st, topk_ids, n, topk,
                       num_experts, perm, tok_sorted, revert, group_sizes, group_offsets, flags);
    return launch_status("moe_dispatch");
  }
  if (n <= kFusedMax) {
    hipLaunchKernelGGL(dispatch_fused_kernel, dim3(1), dim3(kFusedThreads), 0, st, topk_ids, n, topk,
                       num_experts, perm, tok_sorted, revert, group_sizes, group_offsets, flags);
    return launch_status("moe_dispatch");
  }
  hipLaunchKernelGGL(dispatch_count_kernel, dim3((unsigned)nchunks), dim3(kDispThreads), 0, st,
                     topk_ids, n, num_experts, counts, flags);
  hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(1024), 0, st, counts, (int)nchunks,
                     num_experts, group_sizes, group_offsets);
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3((unsigned)nchunks), dim3(kDispThreads), 0, st,
                     topk_ids, n, topk, num_experts, counts, perm, tok_sorted, revert);
  return launch_status("moe_dispatch");
}

static int dispatch_check(const int32_t *topk_ids, int64_t T, int topk, int num_experts, int32_t *perm,
                          int32_t *tok_sorted, int32_t *revert, int32_t *group_sizes) {
  DWM_CHECK_ARG(T >= 0 && topk > 0 && num_experts > 0, "moe_dispatch: bad sizes T=%lld topk=%d E=%d",
                (long long)T, topk, num_experts);
  DWM_UNSUPPORTED_IF(num_experts > kMaxExperts, "moe_dispatch: at most %d experts (got %d)", kMaxExperts,
                     num_experts);
  const int64_t n = T * topk;
  DWM_CHECK_ARG(n < (1ll << 31), "moe_dispatch: T*topk must be < 2^31");
  DWM_CHECK_ARG(group_sizes, "moe_dispatch: null pointer");
  DWM_CHECK_ARG(n == 0 || (topk_ids && perm && tok_sorted && revert), "moe_dispatch: null pointer");
  return DWM_OK;
}

// ---- the allocation-free dispatch ----------------------------------------
// Chunk counters of dwm_moe_dispatch_noalloc: a file-scope device array, one
// copy per GPU, held until the process ends.  Host code uses the address
// hipGetSymbolAddress returns for the current device, never the symbol.
constexpr int64_t kNoAllocWords = 1 << 20;  // 4 MiB: nchunks * (E + 1) int32
static __device__ __align__(256) int32_t scratch[kNoAllocWords];

constexpr int kMaxDevices = 64;
static std::once_flag g_scratch_once[kMaxDevices];
static int32_t *g_scratch[kMaxDevices];
static hipError_t g_scratch_err[kMaxDevices];

// This device's copy of `scratch` (looked up once per device, with the
// device current), or NULL with the error message set.
static int32_t *device_scratch() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("moe_dispatch_noalloc: no usable current device (%s)", hipGetErrorString(e));
    return nullptr;
  }
  std::call_once(g_scratch_once[dev], [dev] {
    void *p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch[dev] = g_scratch_err[dev] == hipSuccess ? (int32_t *)p : nullptr;
  });
  if (!g_scratch[dev])
    set_error("moe_dispatch_noalloc: hipGetSymbolAddress failed on device %d (%s)", dev,
              hipGetErrorString(g_scratch_err[dev]));
  return g_scratch[dev];
}

}  // namespace dwm

using namespace dwm;

extern "C" int dwm_moe_dispatch_workspace_size(int64_t n, int num_experts, int64_t *bytes) {
  clear_error();
  DWM_CHECK_ARG(n >= 0 && num_experts > 0 && bytes, "moe_dispatch_workspace_size: bad arguments");
  DWM_UNSUPPORTED_IF(num_experts > kMaxExperts, "moe_dispatch: at most %d experts", kMaxExperts);
  const int64_t nchunks = (n + kChunk - 1) / kChunk;
  *bytes = nchunks * (num_experts + 1) * 4;
  if (*bytes == 0) *bytes = 4;
  return DWM_OK;
}

extern "C" int dwm_moe_dispatch(const int32_t *topk_ids, int64_t T, int topk, int num_experts,
                                int32_t *perm, int32_t *tok_sorted, int32_t *revert,
                                int32_t *group_sizes, int32_t *group_offsets, int32_t *flags,
                                void *workspace, void *stream) {
  clear_error();
  int rc = dispatch_check(topk_ids, T, topk, num_experts, perm, tok_sorted, revert, group_sizes);
  if (rc != DWM_OK) return rc;
  DWM_CHECK_ARG(workspace, "moe_dispatch: null pointer");
  return dispatch_launch(topk_ids, T * topk, topk, num_experts, perm, tok_sorted, revert, group_sizes,
                         group_offsets, flags, (int32_t *)workspace, as_stream(stream));
}

extern "C" int dwm_moe_dispatch_noalloc(const int32_t *topk_ids, int64_t T, int topk, int num_experts,
                                        int32_t *perm, int32_t *tok_sorted, int32_t *revert,
                                        int32_t *group_sizes, int32_t *group_offsets, int32_t *flags,
                                        void *stream) {
  clear_error();
  int rc = dispatch_check(topk_ids, T, topk, num_experts, perm, tok_sorted, revert, group_sizes);
  if (rc != DWM_OK) return rc;
  const int64_t n = T * topk;
  const int64_t words = (n + kChunk - 1) / kChunk * (int64_t)(num_experts + 1);
  DWM_UNSUPPORTED_IF(n > kFusedMax && words > kNoAllocWords,
                     "moe_dispatch_noalloc: %lld ids over %d experts need %lld counter words, more than the "
                     "%lld of its static scratch (use dwm_moe_dispatch with a workspace)",
                     (long long)n, num_experts, (long long)words, (long long)kNoAllocWords);
  // Only the three-launch path (n > kFusedMax) uses the counters: smaller
  // batches never look the array up, so their first call on a device does
  // no runtime lookup (e.g. inside a stream capture).
  int32_t *counts = nullptr;
  if (n > kFusedMax) {
    counts = device_scratch();
    if (!counts) return DWM_ERR_HIP;
  }
  return dispatch_launch(topk_ids, n, topk, num_experts, perm, tok_sorted, revert, group_sizes, group_offsets,
                         flags, counts, as_stream(stream));
}

static int gather_run(const char *what, const void *src, int64_t src_rows, int64_t row_bytes, const int32_t *idx,
                      int64_t rows, int div, void *out, void *stream) {
  DWM_CHECK_ARG(src_rows >= 0 && row_bytes >= 0 && rows >= 0 && div > 0, "%s: bad sizes", what);
  if (rows == 0 || row_bytes == 0) return DWM_OK;
  DWM_CHECK_ARG(src_rows > 0, "%s: empty source with rows to gather", what);
  DWM_CHECK_ARG(src && idx && out, "%s: null pointer", what);
  const unsigned grid = (unsigned)(rows < 65536 ? rows : 65536);
  hipStream_t st = as_stream(stream);
  const uintptr_t al = (uintptr_t)src | (uintptr_t)out | (uintptr_t)row_bytes;
  if (al % 16 == 0)
    hipLaunchKernelGGL(row_gather_kernel<u32x4_t>, dim3(grid), dim3(256), 0, st, (const char *)src,
                       src_rows, row_bytes, idx, rows, (char *)out, div);
  else if (al % 4 == 0)
    hipLaunchKernelGGL(row_gather_kernel<uint32_t>, dim3(grid), dim3(256), 0, st, (const char *)src,
                       src_rows, row_bytes, idx, rows, (char *)out, div);
  else
    hipLaunchKernelGGL(row_gather_kernel<uint8_t>, dim3(grid), dim3(256), 0, st, (const char *)src,
                       src_rows, row_bytes, idx, rows, (char *)out, div);
  return launch_status(what);
}

extern "C" int dwm_row_gather(const void *src, int64_t src_rows, int64_t row_bytes,
                              const int32_t *idx, int64_t rows, void *out, void *stream) {
  clear_error();
  return gather_run("row_gather", src, src_rows, row_bytes, idx, rows, 1, out, stream);
}

extern "C" int dwm_dispatch_gather(const void *hidden, int64_t T, int64_t row_bytes, const int32_t *argsort,
                                   int64_t rows, int topk, void *out, void *stream) {
  clear_error();
  DWM_CHECK_ARG(topk > 0, "dispatch_gather: topk must be positive (got %d)", topk);
  return gather_run("dispatch_gather", hidden, T, row_bytes, argsort, rows, topk, out, stream);
}

extern "C" int dwm_moe_combine(const void *x, int x_dtype, int64_t x_rows, int64_t H,
                               const int32_t *idx, const void *w, int w_dtype, int64_t T, int topk,
                               void *out, int out_dtype, void *stream) {
  clear_error();
  DWM_CHECK_ARG(x_rows >= 0 && H >= 0 && T >= 0 && topk > 0, "moe_combine: bad sizes");
  DWM_CHECK_ARG((x_dtype == DWM_BF16 || x_dtype == DWM_F32) && (w_dtype == DWM_BF16 || w_dtype == DWM_F32) &&
                    (out_dtype == DWM_BF16 || out_dtype == DWM_F32),
                "moe_combine: bad dtype");
  if (T == 0 || H == 0) return DWM_OK;
  DWM_CHECK_ARG(x_rows > 0, "moe_combine: empty x with tokens to combine");
  DWM_CHECK_ARG(x && idx && w && out, "moe_combine: null pointer");
  const int xf32 = x_dtype == DWM_F32;
  // 16-byte row loads and stores need 8-column multiples and aligned bases.
  const int vec = (H % 8 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)out % 16 == 0);
  const dim3 grid((unsigned)((H + 2047) / 2048), (unsigned)(T < 65535 ? T : 65535));
  hipStream_t st = as_stream(stream);
  const int of32 = out_dtype == DWM_F32;
  if (vec && !xf32) {
    if (of32)
      hipLaunchKernelGGL((combine_bf16_kernel<1>), grid, dim3(256), 0, st, (const uint16_t *)x, x_rows, H, idx, w,
                         w_dtype, T, topk, out);
    else
      hipLaunchKernelGGL((combine_bf16_kernel<0>), grid, dim3(256), 0, st, (const uint16_t *)x, x_rows, H, idx, w,
                         w_dtype, T, topk, out);
    return launch_status("moe_combine");
  }
  if (!xf32 && !of32)
    hipLaunchKernelGGL((combine_kernel<0, 0>), grid, dim3(256), 0, st, x, x_rows, H, idx, w,
                       w_dtype, T, topk, out, vec);
  else if (!xf32 && of32)
    hipLaunchKernelGGL((combine_kernel<0, 1>), grid, dim3(256), 0, st, x, x_rows, H, idx, w,
                       w_dtype, T, topk, out, vec);
  else if (xf32 && !of32)
    hipLaunchKernelGGL((combine_kernel<1, 0>), grid, dim3(256), 0, st, x, x_rows, H, idx, w,
                       w_dtype, T, topk, out, vec);
  else
    hipLaunchKernelGGL((combine_kernel<1, 1>), grid, dim3(256), 0, st, x, x_rows, H, idx, w,
                       w_dtype, T, topk, out, vec);
  return launch_status("moe_combine");
}
