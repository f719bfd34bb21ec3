// Shared parts of the ragged grouped matmul kernels (gmm_fp4.hip: bf16
// MFMA on decoded weights; gmm_mx.hip: scaled MFMA on e4m3 activations):
// the device-side tile list over ragged group_sizes, the fused activation
// and the LDS-staged epilogue of a consumer wave's accumulators (32x32 or
// 16x16 MFMA layouts) for its 64 columns.
#pragma once

#include "common.h"

namespace dwm {

constexpr int kMaxGroups = 1024;
constexpr float kSwigluLimit = 10.0f;  // DeepSeek V4 swiglu_limit of silu_and_mul_with_clamp

// Row tiles are ordered by cost.  A local group of sz rows has sz / MT full
// row tiles and, when sz % MT != 0, one partial tile; a row tile's class is
// its count of CG-row MFMA blocks (1 .. NC = MT / CG), the full tiles' class
// being NC.  Wave 0 computes the exclusive row starts of every group and, per
// class (index 0 = NC blocks, largest first), the exclusive prefix over groups
// of that class's row tiles; s_cls[a * kClsStride + num_groups] is the class
// total.
//
// Balanced groups (bal > 0): a group of n = ceil(sz / MT) row tiles with
// 2 <= n <= bal splits its nb = ceil(sz / CG) blocks evenly instead: tile tt
// holds nb / n blocks, one more for tt < nb % n (only the last block of the
// group is partial).  All n tiles are listed in the class of the largest, and
// a group's entries run (column tile, row tile) with the row tile innermost,
// so the n row tiles of one column tile are adjacent in one XCD's run: they
// run together and stream the expert's weights through that XCD's L2 once
// (a 96-row tile plus a small one would run at different times and each read
// the weights from HBM).  Each row's result depends only on its own lhs row
// and expert (every 16-row block sums K in the same grouping), so the split
// does not change any output bit.
constexpr int kClsStride = kMaxGroups + 1;

template <int MT, int CG>
struct RowSplit {
  // Tiles, blocks and the largest tile's block count of a local group of sz rows.
  int n, nb, top;
  bool bal;
  __device__ __forceinline__ RowSplit(int sz, int bal_max) {  // sz >= 0; no sum that could overflow int32
    n = sz / MT + (sz % MT != 0 ? 1 : 0);
    nb = sz / CG + (sz % CG != 0 ? 1 : 0);
    bal = n >= 2 && n <= bal_max;
    top = bal ? (nb + n - 1) / n : 0;
  }
};

template <int MB, int CG>
__device__ __forceinline__ void tile_classes(const int32_t *group_sizes, int num_groups, int go, int64_t e_local,
                                             int bal, int *s_rowstart, int *s_cls) {
  constexpr int MT = 32 * MB, NC = MT / CG;
  static_assert(NC * CG == MT, "class granularity divides the tile");
  const int lane = threadIdx.x & 63;
  if ((threadIdx.x >> 6) == 0) {
    int row_carry = 0;
    int carry[NC];
#pragma unroll
    for (int a = 0; a < NC; ++a) carry[a] = 0;
    for (int base = 0; base < num_groups; base += 64) {
      const int g = base + lane;
      int sz = g < num_groups ? group_sizes[g] : 0;
      sz = sz > 0 ? sz : 0;
      const bool local = g >= go && (int64_t)g < (int64_t)go + e_local;
      const RowSplit<MT, CG> sp(local ? sz : 0, bal);
      const int n_full = local && !sp.bal ? sz / MT : 0;
      const int rem = local && !sp.bal ? sz % MT : 0;
      const int rem_cls = (rem + CG - 1) / CG;  // 0 when there is no partial tile
      const int ri = wave_inclusive_scan(sz);
      if (g < num_groups) s_rowstart[g] = row_carry + ri - sz;
      row_carry += wave_last(ri);
#pragma unroll
      for (int a = 0; a < NC; ++a) {
        const int cnt = sp.bal ? (sp.top == NC - a ? sp.n : 0)
                               : (a == 0 ? n_full : 0) + (rem_cls == NC - a ? 1 : 0);
        const int ci = wave_inclusive_scan(cnt);
        if (g < num_groups) s_cls[a * kClsStride + g] = carry[a] + ci - cnt;
        carry[a] += wave_last(ci);
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int a = 0; a < NC; ++a) s_cls[a * kClsStride + num_groups] = carry[a];
    }
  }
}

// The block's tile: (local group g, rows row0 .. row0 + rows - 1) x column
// tile nt, of the wide tile width, or of half of it when `narrow`.
struct TileRef {
  int g, rows, nt, narrow;
  int64_t row0;
};
constexpr int kTileInfo = 5;  // s_info: g (-1: no tile), row0, rows, nt, narrow

// The block's work-list entry from the class totals tot(a) (see find_tile):
// the narrow split, then the class `cls` (-1: no tile) of block (xcd, j),
// its entry within the class and the class's column tiles per row tile.
template <int NC, class Tot>
__device__ __forceinline__ void class_entry(Tot tot, int n_tiles, int n_tiles_n, int ncu, int &nsplit, int &cls,
                                            int &per_row, int64_t &entry) {
  nsplit = 0;
  if (n_tiles_n > 0) {
    int64_t spare = (int64_t)ncu;
#pragma unroll
    for (int a = 0; a < NC; ++a) spare -= (int64_t)tot(a) * n_tiles;
    bool open = true;
#pragma unroll
    for (int a = 0; a < NC; ++a) {
      const int64_t extra = (int64_t)tot(a) * (n_tiles_n - n_tiles);
      if (open && extra <= spare) {
        spare -= extra;
        nsplit = a + 1;
      } else {
        open = false;
      }
    }
  }
  const int xcd = blockIdx.x & 7;
  int64_t j = blockIdx.x >> 3;
  cls = -1;
  per_row = n_tiles;
  entry = 0;
#pragma unroll
  for (int a = 0; a < NC; ++a) {
    const int nt_a = a < nsplit ? n_tiles_n : n_tiles;
    const int64_t n_a = (int64_t)tot(a) * nt_a;
    const int64_t per = (n_a + 7) / 8;
    const int64_t lo = xcd * per, hi = min(lo + per, n_a);
    const int64_t len = hi > lo ? hi - lo : 0;
    if (cls < 0) {
      if (j < len) {
        cls = a;
        per_row = nt_a;
        entry = lo + j;
      } else {
        j -= len;
      }
    }
  }
}

// Rows and column tile of entry `entry` (row tile trow of class cls) in
// group g of sz rows starting at row rs, whose class-cls row tiles start at
// cs_g in the class's list.  s_info[1 .. 3] = row0, rows, nt.
template <int MT, int CG>
__device__ __forceinline__ void tile_rows(int sz, int rs, int cs_g, int cls, int trow, int64_t entry, int per_row,
                                          int bal, int *s_info) {
  const RowSplit<MT, CG> sp(sz, bal);
  if (sp.bal) {
    // (column tile, row tile) with the row tile innermost; tile tt starts
    // after tt * base + min(tt, extra) blocks.
    const int64_t local = entry - (int64_t)cs_g * per_row;
    const int tt = (int)(local % sp.n);
    const int base = sp.nb / sp.n, extra = sp.nb % sp.n;
    const int b0 = tt * base + min(tt, extra);
    s_info[1] = rs + CG * b0;
    s_info[2] = min(CG * (base + (tt < extra ? 1 : 0)), sz - CG * b0);
    s_info[3] = (int)(local / sp.n);
  } else {
    // Class 0 holds the full tiles (then a partial one of NC blocks); the
    // other classes hold one partial tile per group.
    const int tt = cls == 0 ? trow - cs_g : sz / MT;
    s_info[1] = rs + tt * MT;
    s_info[2] = min(MT, sz - tt * MT);
    s_info[3] = (int)(entry % per_row);
  }
}

// Wave 0 lists the tiles of at most 64 groups (group g in lane g) without
// LDS: the row starts and the per-class tile counts are independent prefix
// sums (one of sizes, one per class) run side by side in registers, the
// block's group is the one lane whose class range holds its row tile (a
// ballot), and that lane's values are read with readlane.  Same list and
// same tile as the LDS path.
template <int MB, int CG>
__device__ __forceinline__ void pick_tile_lanes(const int32_t *__restrict__ group_sizes, int num_groups, int go,
                                                int64_t e_local, int n_tiles, int n_tiles_n, int ncu, int bal,
                                                int *s_info) {
  constexpr int MT = 32 * MB, NC = MT / CG;
  const int g = threadIdx.x & 63;
  int sz = g < num_groups ? group_sizes[g] : 0;
  sz = sz > 0 ? sz : 0;
  const bool local = g >= go && (int64_t)g < (int64_t)go + e_local;
  const RowSplit<MT, CG> sp(local ? sz : 0, bal);
  const int n_full = local && !sp.bal ? sz / MT : 0;
  const int rem = local && !sp.bal ? sz % MT : 0;
  const int rem_cls = (rem + CG - 1) / CG;  // 0 when there is no partial tile
  int cnt[NC], inc[NC + 1];
#pragma unroll
  for (int a = 0; a < NC; ++a) {
    cnt[a] = sp.bal ? (sp.top == NC - a ? sp.n : 0) : (a == 0 ? n_full : 0) + (rem_cls == NC - a ? 1 : 0);
    inc[a] = cnt[a];
  }
  inc[NC] = sz;
  wave_inclusive_scan_n<NC + 1>(inc);
  int tot[NC];
#pragma unroll
  for (int a = 0; a < NC; ++a) tot[a] = wave_last(inc[a]);
  int nsplit, cls, per_row;
  int64_t entry;
  class_entry<NC>([&](int a) { return tot[a]; }, n_tiles, n_tiles_n, ncu, nsplit, cls, per_row, entry);
  int gsel = -1;
  int trow = 0, ci = 0, cc = 0;
  if (cls >= 0) {
    trow = (int)(entry / per_row);
#pragma unroll
    for (int a = 0; a < NC; ++a)
      if (a == cls) ci = inc[a], cc = cnt[a];
    const uint64_t hit = __ballot(g < num_groups && ci - cc <= trow && trow < ci);
    if (hit) gsel = __ffsll((unsigned long long)hit) - 1;
  }
  const int rs = __builtin_amdgcn_readlane(inc[NC] - sz, gsel < 0 ? 0 : gsel);
  const int szg = __builtin_amdgcn_readlane(sz, gsel < 0 ? 0 : gsel);
  const int csg = __builtin_amdgcn_readlane(ci - cc, gsel < 0 ? 0 : gsel);
  if (g == 0) {
    s_info[0] = gsel;
    s_info[4] = cls >= 0 && cls < nsplit;
    if (gsel >= 0) tile_rows<MT, CG>(szg, rs, csg, cls, trow, entry, per_row, bal, s_info);
  }
}

// Every thread of the block calls this (it holds one block barrier, two
// when there are more than 64 groups).  Work list: the (row tile, column
// tile) pairs of class 0 (NC blocks), then class 1, ... (longest first, so
// the dispatcher's in-order refill of free CUs balances them).  Each class is
// cut into 8 contiguous runs, one per XCD (blocks equal mod 8 run on one
// XCD), so a row tile's column tiles share that XCD's L2.
//
// Narrow split (n_tiles_n > 0): when the wide tiles leave some of the ncu CUs
// idle, the costliest classes are cut into column tiles of half the width
// (n_tiles_n per row tile), whole classes at a time and only while the tile
// count stays within ncu, so the longest tiles of a one-round launch get the
// idle CUs.  Returns false when the block has no tile.
template <int MB, int CG, int THREADS>
__device__ __forceinline__ bool find_tile(const int32_t *__restrict__ group_sizes, int num_groups, int go,
                                          int64_t e_local, int64_t M, int n_tiles, int n_tiles_n, int ncu, int bal,
                                          int *s_rowstart, int *s_cls, int *s_info, TileRef &ref) {
  constexpr int MT = 32 * MB, NC = MT / CG;
  const int tid = threadIdx.x;
  if (num_groups <= 64) {
    if ((tid >> 6) == 0)
      pick_tile_lanes<MB, CG>(group_sizes, num_groups, go, e_local, n_tiles, n_tiles_n, ncu, bal, s_info);
  } else {
    tile_classes<MB, CG>(group_sizes, num_groups, go, e_local, bal, s_rowstart, s_cls);
    if (tid == 0) s_info[0] = -1;
    __syncthreads();
    int nsplit, cls, per_row;
    int64_t entry;
    class_entry<NC>([&](int a) { return s_cls[a * kClsStride + num_groups]; }, n_tiles, n_tiles_n, ncu, nsplit, cls,
                    per_row, entry);
    if (tid == 0) s_info[4] = cls >= 0 && cls < nsplit;
    if (cls >= 0) {
      const int trow = (int)(entry / per_row);
      const int *const cs = s_cls + cls * kClsStride;
      for (int g = tid; g < num_groups; g += THREADS) {
        if (cs[g] <= trow && trow < cs[g + 1]) {
          s_info[0] = g;
          tile_rows<MT, CG>(group_sizes[g], s_rowstart[g], cs[g], cls, trow, entry, per_row, bal, s_info);
        }
      }
    }
  }
  __syncthreads();  // also retires the class reads before the stages overwrite them
  ref.g = s_info[0];
  if (ref.g < 0) return false;
  ref.nt = s_info[3];
  ref.narrow = s_info[4];
  ref.row0 = s_info[1];
  // group_sizes lives on the device and is not checked by the host: sizes
  // whose sum leaves int32 would give row starts outside [0, M).  Such tiles
  // are skipped, so no tile reads or writes a row outside [0, M).
  if (ref.row0 < 0 || ref.row0 >= M) return false;
  ref.rows = (int)min((int64_t)s_info[2], M - ref.row0);
  return ref.rows > 0;
}

// The fused activation of one (gate, up) accumulator pair, in f32 (the
// activations of apply_act_fn, patches/tpu-inference-experimental/
// fused-moe-fp4/0901-...:57-66).
__device__ __forceinline__ float act_pair(int act, float gate, float up) {
  switch (act) {
    case DWM_ACT_SILU_MUL_CLAMP: {  // DeepSeek V4, swiglu_limit 10
      const float g = fminf(gate, kSwigluLimit);
      const float u = fminf(fmaxf(up, -kSwigluLimit), kSwigluLimit);
      return g / (1.0f + expf(-g)) * u;
    }
    case DWM_ACT_SILU_MUL:
      return gate / (1.0f + expf(-gate)) * up;
    case DWM_ACT_GELU_TANH_MUL: {  // jax.nn.gelu's default (tanh) form
      const float inner = 0.7978845608028654f * (gate + 0.044715f * (gate * gate * gate));
      return gate * (0.5f * (1.0f + tanhf(inner))) * up;
    }
    case DWM_ACT_SWIGLUOAI: {  // GPT-OSS: alpha 1.702, limit 7
      const float g = fminf(gate, 7.0f);
      const float u = fminf(fmaxf(up, -7.0f), 7.0f);
      return g / (1.0f + expf(-1.702f * g)) * (u + 1.0f);
    }
    default:
      return 0.0f;
  }
}

__device__ __forceinline__ float bias_at(const void *bias, int bias_bf16, int64_t i) {
  return bias_bf16 ? bf16_bits_to_f32(((const uint16_t *)bias)[i]) : ((const float *)bias)[i];
}

// Stores 8 consecutive output values of one row (16-byte bf16 or 2 x 16-byte f32
// stores), as streaming (non-temporal) vector stores: the output is read back
// only by a later kernel.
__device__ __forceinline__ void store8(void *__restrict__ out, int64_t o, const float *v, int out_f32) {
  if (out_f32) {
    u32x4_t lo, hi;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = __builtin_bit_cast(uint32_t, v[i]);
      hi[i] = __builtin_bit_cast(uint32_t, v[4 + i]);
    }
    __builtin_nontemporal_store(lo, (u32x4_t *)((float *)out + o));
    __builtin_nontemporal_store(hi, (u32x4_t *)((float *)out + o + 4));
  } else {
    u32x4_t p;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      p[i] = f32x2_to_bf16x2_bits(v[2 * i], v[2 * i + 1]);
    __builtin_nontemporal_store(p, (u32x4_t *)((uint16_t *)out + o));
  }
}

// Writes one consumer wave's accumulators acc[mb][j] (the 32 x 32 MFMA
// layout: register r of lane (c32, h) is row 8 (r / 4) + 4 h + r % 4, column
// c32 of 32-column block j) for its 64 packed columns col0 .. col0 + 63
// through a private LDS region `ep` of 32 rows x ES floats, 32 rows at a
// time, as whole 8-column runs of a row.  `bias` (NULL, or this expert's
// [N] row, f32 or bf16) is added to the f32 accumulators first.  With ACT,
// block 0 holds the gate and block 1 the up projection of the same 32 output
// columns (gate_up prepack: packed column 64 g + 32 j + c is source column
// j N/2 + 32 g + c) and `act` (DWM_ACT_*) combines them.
template <int AM, bool ACT, int ES>
__device__ __forceinline__ void store_tile(const f32x16_t (&acc)[AM][2], float *ep, int64_t row0, int rows,
                                           int64_t col0, int N, void *__restrict__ out, int out_f32,
                                           const void *__restrict__ bias, int bias_bf16, int act) {
  const int lane = threadIdx.x & 63, c32 = lane & 31, h = lane >> 5;
  constexpr int CO = ACT ? 32 : 64;  // output columns of this wave
  const int64_t n_out = ACT ? N / 2 : N;
  const int64_t ocol0 = ACT ? col0 / 2 : col0;
  // The bias of this lane's two accumulator columns (source column order);
  // -0.0f without a bias: x + -0.0f is x for every accumulator value (f32
  // denormals are kept), so no per-value select is needed.
  float b0 = -0.0f, b1 = -0.0f;
  if (bias) {
    const int64_t s0 = ACT ? col0 / 2 + c32 : col0 + c32;
    const int64_t s1 = ACT ? N / 2 + col0 / 2 + c32 : col0 + 32 + c32;
    if (s0 < N) b0 = bias_at(bias, bias_bf16, s0);
    if (s1 < N) b1 = bias_at(bias, bias_bf16, s1);
  }
#pragma unroll
  for (int mb = 0; mb < AM; ++mb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int lr = 8 * (r >> 2) + 4 * h + (r & 3);
      const float v0 = acc[mb][0][r] + b0;
      const float v1 = acc[mb][1][r] + b1;
      if constexpr (ACT) {
        ep[lr * ES + c32] = act_pair(act, v0, v1);
      } else {
        ep[lr * ES + c32] = v0;
        ep[lr * ES + 32 + c32] = v1;
      }
    }
    // Lane q of chunk i covers row q / (CO / 8), columns 8 (q % (CO / 8)) .. + 7.
#pragma unroll
    for (int i = 0; i < 32 * CO / 8 / 64; ++i) {
      const int q = lane + 64 * i;
      const int lr = q / (CO / 8), c8 = q % (CO / 8);
      const int row = mb * 32 + lr;
      const int64_t col = ocol0 + 8 * c8;
      float v[8];
      const f32x4_t lo = *(const f32x4_t *)(ep + lr * ES + 8 * c8);
      const f32x4_t hi = *(const f32x4_t *)(ep + lr * ES + 8 * c8 + 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[k] = lo[k];
        v[4 + k] = hi[k];
      }
      if (row < rows && col < n_out) store8(out, (row0 + row) * n_out + col, v, out_f32);
    }
  }
}

// Writes one consumer wave's 16x16x32 MFMA accumulators for NH 16-row
// blocks (register r of acc[hb][u] in lane (c16, q) is tile row 16 hb + 4 q +
// r, column 16 u + c16 of the wave's 64 packed columns col0 .. col0 + 63)
// through `ep` like store_tile, 16 rows at a time.  With ACT, acc[hb][u] and
// acc[hb][u + 2] are the gate and up projections of output column
// 16 u + c16 (packed columns 32 j + c hold source column j N / 2 + col0 / 2 + c).
template <int NH, bool ACT, int ES>
__device__ __forceinline__ void store_halves(const f32x4_t (&acc)[NH][4], float *ep, int64_t row0, int rows,
                                             int64_t col0, int N, void *__restrict__ out, int out_f32,
                                             const void *__restrict__ bias, int bias_bf16, int act) {
  const int lane = threadIdx.x & 63, c16 = lane & 15, q = lane >> 4;
  constexpr int CO = ACT ? 32 : 64;
  const int64_t n_out = ACT ? N / 2 : N;
  const int64_t ocol0 = ACT ? col0 / 2 : col0;
  float b[4] = {-0.0f, -0.0f, -0.0f, -0.0f};  // no bias: x + -0.0f is x (see store_tile)
  if (bias) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = 16 * (u & 1) + c16;  // column within its 32-column block
      const int64_t s = ACT ? (u < 2 ? col0 / 2 + c : N / 2 + col0 / 2 + c) : col0 + 16 * u + c16;
      if (s < N) b[u] = bias_at(bias, bias_bf16, s);
    }
  }
#pragma unroll
  for (int hb = 0; hb < NH; ++hb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int lr = 4 * q + r;
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = acc[hb][u][r] + b[u];
      if constexpr (ACT) {
        ep[lr * ES + c16] = act_pair(act, v[0], v[2]);
        ep[lr * ES + 16 + c16] = act_pair(act, v[1], v[3]);
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) ep[lr * ES + 16 * u + c16] = v[u];
      }
    }
    // Lane p of chunk i covers row p / (CO / 8), columns 8 (p % (CO / 8)) .. + 7.
#pragma unroll
    for (int i = 0; i < 16 * CO / 8 / 64; ++i) {
      const int p = lane + 64 * i;
      const int lr = p / (CO / 8), c8 = p % (CO / 8);
      const int row = 16 * hb + lr;
      const int64_t col = ocol0 + 8 * c8;
      float v[8];
      const f32x4_t lo = *(const f32x4_t *)(ep + lr * ES + 8 * c8);
      const f32x4_t hi = *(const f32x4_t *)(ep + lr * ES + 8 * c8 + 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[k] = lo[k];
        v[4 + k] = hi[k];
      }
      if (row < rows && col < n_out) store8(out, (row0 + row) * n_out + col, v, out_f32);
    }
  }
}

// Epilogue inputs every gmm kernel passes through to store_tile.
struct GmmEpilogue {
  const void *bias;  // [E_local, N] (f32 or bf16) or NULL
  int bias_bf16;
  int act;           // DWM_ACT_*
};

// The bias row of local expert e (NULL when there is no bias).
__device__ __forceinline__ const void *expert_bias(const GmmEpilogue &ep, int64_t e, int N) {
  return ep.bias ? (const void *)((const uint8_t *)ep.bias + e * (int64_t)N * (ep.bias_bf16 ? 2 : 4)) : nullptr;
}

// Zeroes the rows outside the local groups (zero_initialize); host side.
int launch_gmm_zero_rows(const int32_t *group_sizes, int num_groups, const int32_t *group_offset, int64_t e_local,
                         int64_t M, int64_t n_out, void *out, int elem_bytes, hipStream_t st);

// The grouped matmuls behind the C ABI (host side): bf16 lhs (gmm_fp4.hip)
// and MX lhs (gmm_mx.hip).  Arguments as dwm_gmm_fp4_ex, checked by the
// caller; `gated` = the activation reads gate/up pairs.
int launch_gmm_bf16(const uint16_t *lhs, const int32_t *row_idx, int64_t lhs_rows, int64_t M, int64_t K,
                    const uint8_t *weight, const uint8_t *scale, const int32_t *group_sizes, int num_groups,
                    const int32_t *group_offset, int64_t E_local, int64_t N, void *out, int out_f32, bool gated,
                    const GmmEpilogue &ep, hipStream_t st);
int launch_gmm_mx(const uint8_t *lhs, const uint8_t *lhs_scale, const int32_t *row_idx, int64_t lhs_rows, int64_t M,
                  int64_t K, const uint8_t *weight, const uint8_t *scale, const int32_t *group_sizes, int num_groups,
                  const int32_t *group_offset, int64_t E_local, int64_t N, void *out, int out_f32, bool gated,
                  const GmmEpilogue &ep, hipStream_t st, bool lhs_fp4 = false);

}  // namespace dwm
