// Ragged grouped matmul with FP4 (e2m1 + e8m0 block-32) weights, bf16
// activations, f32 accumulation: the tokamax gmm_v2 rhs_fp4_codes path
// (patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:58-66, :100-151).
//
// Work decomposition: a block owns one (local group, 32*MB-row tile) x
// (32*NB*4-column tile).  Tiles are enumerated on the device from
// group_sizes (no host sync): blockIdx.y is a tile slot, blockIdx.x the
// column tile; slots past the last tile exit at once, empty groups own no
// slot and cost no weight traffic.
//
// Per 64-deep K step: the block stages its [rows x 64] bf16 lhs tile in LDS
// (double buffered, one barrier per step); each wave streams NB 1 KiB weight
// chunks (16 B per lane, prepacked K-major, see fp4.hip), decodes them in
// registers with the gfx950 fp4 -> bf16 converter (which applies the e8m0
// scale exactly), and issues bf16 MFMA 32x32x16 for every active 32-row
// block.  The weight dequant is exact (e2m1 x power of two fits bf16), so the
// products equal the reference's bf16(decode(q)) * bf16(scale) operands.
#include "common.h"

namespace dwm {

constexpr int kGmmThreads = 256;  // 4 waves
constexpr int kMaxGroups = 1024;
constexpr int kLdsRow = 72;       // bf16 per LDS row: 64 + 8 pad (144 B keeps ds_read_b128 conflict-free)

// Block-wide: exclusive row starts and tile starts of every group, computed
// by wave 0.  s_tilestart[num_groups] receives the tile total.
template <int MT>
__device__ __forceinline__ void group_prefix(const int32_t *group_sizes, int num_groups, int go,
                                             int64_t e_local, int *s_rowstart, int *s_tilestart) {
  const int lane = threadIdx.x & 63;
  if ((threadIdx.x >> 6) == 0) {
    int row_carry = 0, tile_carry = 0;
    for (int base = 0; base < num_groups; base += 64) {
      const int g = base + lane;
      int sz = g < num_groups ? group_sizes[g] : 0;
      sz = sz > 0 ? sz : 0;
      const bool local = g >= go && (int64_t)g < (int64_t)go + e_local;
      const int nt = local ? (sz + MT - 1) / MT : 0;
      const int ri = wave_inclusive_scan(sz);
      const int ti = wave_inclusive_scan(nt);
      if (g < num_groups) {
        s_rowstart[g] = row_carry + ri - sz;
        s_tilestart[g] = tile_carry + ti - nt;
      }
      row_carry += __shfl(ri, 63, 64);
      tile_carry += __shfl(ti, 63, 64);
    }
    if (lane == 0) s_tilestart[num_groups] = tile_carry;
  }
}

template <int MB, int NB>
__global__ __launch_bounds__(kGmmThreads) void gmm_fp4_bf16_kernel(
    const uint16_t *__restrict__ lhs, int64_t M, int K, const uint8_t *__restrict__ wpk,
    const uint8_t *__restrict__ spk, const int32_t *__restrict__ group_sizes, int num_groups,
    const int32_t *__restrict__ group_offset, int64_t e_local, int N, void *__restrict__ out,
    int out_f32) {
  constexpr int MT = 32 * MB;
  __shared__ int s_rowstart[kMaxGroups];
  __shared__ int s_tilestart[kMaxGroups + 1];
  __shared__ int s_info[3];
  __shared__ __attribute__((aligned(16))) uint16_t s_a[2][MT * kLdsRow];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int go = group_offset ? group_offset[0] : 0;
  group_prefix<MT>(group_sizes, num_groups, go, e_local, s_rowstart, s_tilestart);
  if (tid == 0) s_info[0] = -1;
  __syncthreads();
  const int slot = blockIdx.y;
  if (slot >= s_tilestart[num_groups]) return;  // block-uniform
  for (int g = tid; g < num_groups; g += kGmmThreads) {
    if (s_tilestart[g] <= slot && slot < s_tilestart[g + 1]) {
      const int t = slot - s_tilestart[g];
      const int sz = group_sizes[g];
      s_info[0] = g;
      s_info[1] = s_rowstart[g] + t * MT;
      s_info[2] = min(MT, sz - t * MT);
    }
  }
  __syncthreads();
  const int g = s_info[0];
  if (g < 0) return;
  const int64_t row0 = s_info[1];
  if (row0 >= M) return;
  const int rows = (int)min((int64_t)s_info[2], M - row0);
  const int act_mb = (rows + 31) >> 5;
  const int64_t e = g - go;

  const int N32 = N >> 5, KB = K >> 6, KB4 = (KB + 3) >> 2;
  const int nb0 = blockIdx.x * (NB * 4) + wave * NB;
  const uint8_t *wp[NB];
  const uint8_t *sp[NB];
  bool nvalid[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int nbg = nb0 + j;
    nvalid[j] = nbg < N32;
    const int64_t nbc = nvalid[j] ? nbg : 0;
    wp[j] = wpk + ((e * N32 + nbc) * KB) * 1024 + lane * 16;
    sp[j] = spk + ((e * N32 + nbc) * KB4) * 256 + lane * 4;
  }

  f32x16_t acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][j][r] = 0.0f;

  // lhs tile staging: MT rows x 8 chunks of 16 B; thread handles MB chunks.
  const int a_rows = act_mb * 32;
  u32x4_t areg[MB];
  auto load_a = [&](int kb) {
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int c = tid + i * kGmmThreads;
      const int r = c >> 3, col8 = c & 7;
      if (r < a_rows) {
        int64_t grow = row0 + r;
        if (grow >= M) grow = M - 1;  // rows past the tile feed only unstored outputs
        areg[i] = *(const u32x4_t *)(lhs + grow * K + (int64_t)kb * 64 + col8 * 8);
      }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int c = tid + i * kGmmThreads;
      const int r = c >> 3, col8 = c & 7;
      if (r < a_rows) *(u32x4_t *)(&s_a[buf][r * kLdsRow + col8 * 8]) = areg[i];
    }
  };

  u32x4_t wcur[NB], wnxt[NB];
  uint32_t scur[NB], snxt[NB];
  load_a(0);
  store_a(0);
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    wcur[j] = *(const u32x4_t *)(wp[j]);
    scur[j] = *(const uint32_t *)(sp[j]);
  }
  __syncthreads();

  const int arow = lane & 31, acol = 32 * (lane >> 5);
  for (int kb = 0; kb < KB; ++kb) {
    const int buf = kb & 1;
    const bool more = kb + 1 < KB;
    if (more) {
      load_a(kb + 1);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        wnxt[j] = *(const u32x4_t *)(wp[j] + (int64_t)(kb + 1) * 1024);
        snxt[j] = ((kb + 1) & 3) == 0 ? *(const uint32_t *)(sp[j] + (int64_t)((kb + 1) >> 2) * 256)
                                      : scur[j];
      }
    }
    // Decode this step's weights: 32 K values per lane per n-block.
    u32x4_t bfrag[NB][4];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const float sc = e8m0_to_f32(scur[j] >> (8 * (kb & 3)));
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t w = wcur[j][s];
        bfrag[j][s][0] = cvt_fp4x2_bf16<0>(w, sc);
        bfrag[j][s][1] = cvt_fp4x2_bf16<1>(w, sc);
        bfrag[j][s][2] = cvt_fp4x2_bf16<2>(w, sc);
        bfrag[j][s][3] = cvt_fp4x2_bf16<3>(w, sc);
      }
    }
    const uint16_t *abase = &s_a[buf][arow * kLdsRow + acol];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        if (mb < act_mb) {
          const u32x4_t a = *(const u32x4_t *)(abase + mb * 32 * kLdsRow + 8 * s);
#pragma unroll
          for (int j = 0; j < NB; ++j)
            acc[mb][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, bfrag[j][s]),
                acc[mb][j], 0, 0, 0);
        }
      }
    }
    if (more) store_a(buf ^ 1);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      wcur[j] = wnxt[j];
      scur[j] = snxt[j];
    }
  }

  // Epilogue: C layout of mfma 32x32: reg r -> row 8*(r/4) + 4*(lane/32) + r%4, col lane%32.
  const int hrow = 4 * (lane >> 5);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    if (mb >= act_mb) continue;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (!nvalid[j]) continue;
      const int64_t col = (int64_t)(nb0 + j) * 32 + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lrow = mb * 32 + 8 * (r >> 2) + hrow + (r & 3);
        if (lrow < rows) {
          const int64_t o = (row0 + lrow) * N + col;
          if (out_f32) ((float *)out)[o] = acc[mb][j][r];
          else ((uint16_t *)out)[o] = f32_to_bf16_bits(acc[mb][j][r]);
        }
      }
    }
  }
}

// zero_initialize: zero rows outside [start(go), start(go + E_local)).
__global__ __launch_bounds__(256) void gmm_zero_rows_kernel(const int32_t *group_sizes, int num_groups,
                                                            const int32_t *group_offset, int64_t e_local,
                                                            int64_t M, int64_t N, void *out,
                                                            int elem_bytes) {
  __shared__ int64_t s_lohi[2];
  const int lane = threadIdx.x & 63;
  if ((threadIdx.x >> 6) == 0) {
    const int go = group_offset ? group_offset[0] : 0;
    int64_t lo = 0, hi = 0;
    for (int base = 0; base < num_groups; base += 64) {
      const int g = base + lane;
      int sz = g < num_groups ? group_sizes[g] : 0;
      sz = sz > 0 ? sz : 0;
      lo += wave_sum(g < go ? sz : 0);
      hi += wave_sum((int64_t)g < (int64_t)go + e_local ? sz : 0);
    }
    if (lane == 0) {
      s_lohi[0] = lo;
      s_lohi[1] = hi;
    }
  }
  __syncthreads();
  const int64_t lo = s_lohi[0], hi = s_lohi[1];
  const int64_t r0 = (int64_t)blockIdx.x * 64;
  const int64_t row_words = N * elem_bytes / 4;  // N*elem_bytes is a multiple of 64
  for (int64_t r = r0; r < r0 + 64 && r < M; ++r) {
    if (r >= lo && r < hi) continue;
    uint32_t *p = (uint32_t *)((char *)out + r * N * elem_bytes);
    for (int64_t i = threadIdx.x; i < row_words; i += blockDim.x) p[i] = 0u;
  }
}

template <int MB, int NB>
static int launch_gmm(const uint16_t *lhs, int64_t M, int64_t K, const uint8_t *w, const uint8_t *s,
                      const int32_t *gs, int ng, const int32_t *go, int64_t e_local, int64_t N,
                      void *out, int out_f32, hipStream_t st) {
  constexpr int MT = 32 * MB, NT = 32 * NB * 4;
  const int64_t gx = (N + NT - 1) / NT;
  const int64_t gy = (M + MT - 1) / MT + e_local;
  DWM_UNSUPPORTED_IF(gy > 65535, "gmm_fp4: too many row tiles (%lld)", (long long)gy);
  hipLaunchKernelGGL((gmm_fp4_bf16_kernel<MB, NB>), dim3((unsigned)gx, (unsigned)gy), dim3(kGmmThreads),
                     0, st, lhs, M, (int)K, w, s, gs, ng, go, e_local, (int)N, out, out_f32);
  return launch_status("gmm_fp4");
}

}  // namespace dwm

using namespace dwm;

extern "C" int dwm_gmm_fp4(const uint16_t *lhs, int64_t M, int64_t K, const uint8_t *weight,
                           const uint8_t *scale, const int32_t *group_sizes, int num_groups,
                           const int32_t *group_offset, int64_t E_local, int64_t N, void *out,
                           int out_dtype, int zero_init, void *stream) {
  clear_error();
  DWM_CHECK_ARG(M >= 0 && K > 0 && N > 0 && E_local >= 0 && num_groups >= 0,
                "gmm_fp4: bad sizes M=%lld K=%lld N=%lld E_local=%lld groups=%d", (long long)M,
                (long long)K, (long long)N, (long long)E_local, num_groups);
  DWM_CHECK_ARG(out_dtype == DWM_BF16 || out_dtype == DWM_F32, "gmm_fp4: bad out dtype %d", out_dtype);
  DWM_UNSUPPORTED_IF(K % 64 != 0 || N % 32 != 0, "gmm_fp4: K %% 64 == 0 and N %% 32 == 0 required");
  DWM_UNSUPPORTED_IF(num_groups > kMaxGroups, "gmm_fp4: at most %d groups (got %d)", kMaxGroups, num_groups);
  DWM_UNSUPPORTED_IF(K > (1 << 30) || N > (1 << 30), "gmm_fp4: K, N must be < 2^30");
  if (M == 0) return DWM_OK;
  DWM_CHECK_ARG(lhs && out && (num_groups == 0 || group_sizes), "gmm_fp4: null pointer");
  DWM_CHECK_ARG(E_local == 0 || (weight && scale), "gmm_fp4: null weight pointer");
  DWM_CHECK_ARG((uintptr_t)lhs % 16 == 0 && (uintptr_t)weight % 16 == 0 && (uintptr_t)scale % 4 == 0,
                "gmm_fp4: lhs and weight must be 16-byte aligned, scale 4-byte aligned");
  hipStream_t st = as_stream(stream);
  const int elem = out_dtype == DWM_F32 ? 4 : 2;
  if (zero_init) {
    hipLaunchKernelGGL(gmm_zero_rows_kernel, dim3((unsigned)((M + 63) / 64)), dim3(256), 0, st,
                       group_sizes, num_groups, group_offset, E_local, M, N, out, elem);
    int rc = launch_status("gmm_fp4 zero rows");
    if (rc != DWM_OK) return rc;
  }
  if (E_local == 0 || num_groups == 0) return DWM_OK;
  const int out_f32 = out_dtype == DWM_F32;
  // Column tile: 128 columns when groups are decode-sized (spreads the
  // weight stream over more blocks), 256 otherwise.
  const int64_t avg_rows = M / (E_local < num_groups ? E_local : num_groups);
  if (avg_rows <= 256)
    return launch_gmm<4, 1>(lhs, M, K, weight, scale, group_sizes, num_groups, group_offset, E_local,
                            N, out, out_f32, st);
  return launch_gmm<4, 2>(lhs, M, K, weight, scale, group_sizes, num_groups, group_offset, E_local, N,
                          out, out_f32, st);
}
