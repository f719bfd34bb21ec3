// Ragged grouped matmul with FP4 (e2m1 + e8m0 block-32) weights, bf16
// activations, f32 accumulation: the tokamax gmm_v2 rhs_fp4_codes path
// (patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:58-66, :100-151).
//
// Work decomposition: a block (4 waves) owns one (local group, 16*MB-row
// tile) x (64*NBW-column tile); each wave owns NBW 16-column blocks of it.
// Tiles are enumerated on the device from group_sizes (no host sync): the
// tile total is (row tiles of every local group) x (column tiles); empty
// groups own no tile and cost no weight traffic.  Blocks whose index is equal
// mod 8 run on one XCD (the dispatcher's round robin), so each XCD gets a
// contiguous run of tiles -- consecutive column tiles of the same row tile --
// and the group's lhs rows stay in that XCD's L2.
//
// Per 128-deep K step: the block stages its [rows x 128] bf16 lhs tile in
// LDS (double buffered, padded rows, one barrier per step); each wave holds a
// DEPTH-step register ring of its weight chunks (1 KiB per 16 columns x 128 K,
// prepacked, see fp4.hip), decodes the current step in registers with the
// gfx950 fp4 -> bf16 converter (which applies the e8m0 scale exactly) and
// issues bf16 MFMA 16x16x32 for every 16-row block that holds rows.  The
// dequantised weights are exact (e2m1 x power of two fits bf16), so the
// products equal the reference's bf16(decode(q)) * bf16(scale) operands.
#include "common.h"

namespace dwm {

constexpr int kGmmThreads = 256;  // 4 waves
constexpr int kMaxGroups = 1024;
constexpr int kLdsRow = 136;      // bf16 per LDS row: 128 + 8 pad (272 B: conflict-free ds_read_b128)

// Block-wide: exclusive row starts and row-tile starts of every group,
// computed by wave 0.  s_tilestart[num_groups] receives the row-tile total.
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

template <int MB, int NBW, int DEPTH>
__global__ __launch_bounds__(kGmmThreads) void gmm_fp4_bf16_kernel(
    const uint16_t *__restrict__ lhs, int64_t M, int K, const uint8_t *__restrict__ wpk,
    const uint8_t *__restrict__ spk, const int32_t *__restrict__ group_sizes, int num_groups,
    const int32_t *__restrict__ group_offset, int64_t e_local, int N, void *__restrict__ out,
    int out_f32) {
  constexpr int MT = 16 * MB;
  constexpr int NT = 64 * NBW;
  __shared__ int s_rowstart[kMaxGroups];
  __shared__ int s_tilestart[kMaxGroups + 1];
  __shared__ int s_info[3];
  __shared__ __attribute__((aligned(16))) uint16_t s_a[2][MT * kLdsRow];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int go = group_offset ? group_offset[0] : 0;
  group_prefix<MT>(group_sizes, num_groups, go, e_local, s_rowstart, s_tilestart);
  if (tid == 0) s_info[0] = -1;
  __syncthreads();
  const int n_tiles = (N + NT - 1) / NT;
  const int64_t total = (int64_t)s_tilestart[num_groups] * n_tiles;
  const int64_t per_xcd = (total + 7) / 8;
  const int64_t j_x = blockIdx.x >> 3;
  if (j_x >= per_xcd) return;  // block-uniform
  const int64_t t = (int64_t)(blockIdx.x & 7) * per_xcd + j_x;
  if (t >= total) return;
  const int trow = (int)(t / n_tiles), nt = (int)(t % n_tiles);
  for (int g = tid; g < num_groups; g += kGmmThreads) {
    if (s_tilestart[g] <= trow && trow < s_tilestart[g + 1]) {
      const int tt = trow - s_tilestart[g];
      s_info[0] = g;
      s_info[1] = s_rowstart[g] + tt * MT;
      s_info[2] = min(MT, group_sizes[g] - tt * MT);
    }
  }
  __syncthreads();
  const int g = s_info[0];
  if (g < 0) return;
  const int64_t row0 = s_info[1];
  if (row0 >= M) return;
  const int rows = (int)min((int64_t)s_info[2], M - row0);
  const int act_mb = (rows + 15) >> 4;
  const int64_t e = g - go;

  const int N16 = N >> 4, KB = K >> 7, KB4 = (KB + 3) >> 2;
  const int nb0 = nt * (NBW * 4) + wave * NBW;
  const uint8_t *wp[NBW];
  const uint8_t *sp[NBW];
  bool nvalid[NBW];
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    const int nbg = nb0 + j;
    nvalid[j] = nbg < N16;
    const int64_t nbc = nvalid[j] ? nbg : 0;
    wp[j] = wpk + ((e * N16 + nbc) * KB) * 1024 + lane * 16;
    sp[j] = spk + ((e * N16 + nbc) * KB4) * 256 + lane * 4;
  }

  f32x4_t acc[MB][NBW];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[mb][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // lhs tile staging: 16*act_mb rows x 16 chunks of 16 B; chunk tid + 256*i
  // is row 16*i + tid/16, so the row-block test is block-uniform.
  const int srow = tid >> 4, scol = (tid & 15) * 8;
  u32x4_t areg[MB];
  auto load_a = [&](int kb) {
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      if (i < act_mb) {
        int64_t grow = row0 + 16 * i + srow;
        if (grow >= M) grow = M - 1;  // rows past the tile feed only unstored outputs
        areg[i] = *(const u32x4_t *)(lhs + grow * K + (int64_t)kb * 128 + scol);
      }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < MB; ++i)
      if (i < act_mb) *(u32x4_t *)(&s_a[buf][(16 * i + srow) * kLdsRow + scol]) = areg[i];
  };

  u32x4_t wbuf[DEPTH][NBW];
  uint32_t sbuf[DEPTH][NBW];
  auto load_w = [&](int slot, int kb) {
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      wbuf[slot][j] = *(const u32x4_t *)(wp[j] + (int64_t)kb * 1024);
      sbuf[slot][j] = sp[j][(int64_t)(kb >> 2) * 256 + (kb & 3)];
    }
  };

  load_a(0);
#pragma unroll
  for (int d = 0; d < DEPTH; ++d)
    if (d < KB) load_w(d, d);
  store_a(0);
  __syncthreads();

  const int arow = lane & 15, acol = 32 * (lane >> 4);
  for (int kb0 = 0; kb0 < KB; kb0 += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int kb = kb0 + d;
      if (kb < KB) {
        const int buf = kb & 1;
        const bool more = kb + 1 < KB;
        if (more) load_a(kb + 1);
        u32x4_t wcur[NBW];
        float sc[NBW];
#pragma unroll
        for (int j = 0; j < NBW; ++j) {
          wcur[j] = wbuf[d][j];
          sc[j] = e8m0_to_f32(sbuf[d][j]);
        }
        if (kb + DEPTH < KB) load_w(d, kb + DEPTH);
        const uint16_t *abase = &s_a[buf][arow * kLdsRow + acol];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          u32x4_t bfrag[NBW];
#pragma unroll
          for (int j = 0; j < NBW; ++j) {
            const uint32_t w = wcur[j][s];
            bfrag[j][0] = cvt_fp4x2_bf16<0>(w, sc[j]);
            bfrag[j][1] = cvt_fp4x2_bf16<1>(w, sc[j]);
            bfrag[j][2] = cvt_fp4x2_bf16<2>(w, sc[j]);
            bfrag[j][3] = cvt_fp4x2_bf16<3>(w, sc[j]);
          }
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            if (mb < act_mb) {
              const u32x4_t a = *(const u32x4_t *)(abase + mb * 16 * kLdsRow + 8 * s);
#pragma unroll
              for (int j = 0; j < NBW; ++j)
                acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, bfrag[j]), acc[mb][j],
                    0, 0, 0);
            }
          }
        }
        if (more) store_a(buf ^ 1);
        __syncthreads();
      }
    }
  }

  // Epilogue: C layout of mfma 16x16: reg r -> row 4*(lane/16) + r, col lane%16.
  const int qrow = 4 * (lane >> 4);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    if (mb >= act_mb) continue;
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      if (!nvalid[j]) continue;
      const int64_t col = (int64_t)(nb0 + j) * 16 + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int lrow = mb * 16 + qrow + r;
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
  const int64_t row_words = N * elem_bytes / 4;  // N % 16 == 0: whole 32-bit words
  for (int64_t r = r0; r < r0 + 64 && r < M; ++r) {
    if (r >= lo && r < hi) continue;
    uint32_t *p = (uint32_t *)((char *)out + r * N * elem_bytes);
    for (int64_t i = threadIdx.x; i < row_words; i += blockDim.x) p[i] = 0u;
  }
}

template <int MB, int NBW, int DEPTH>
static int launch_gmm(const uint16_t *lhs, int64_t M, int64_t K, const uint8_t *w, const uint8_t *s,
                      const int32_t *gs, int ng, const int32_t *go, int64_t e_local, int64_t N,
                      void *out, int out_f32, hipStream_t st) {
  constexpr int MT = 16 * MB, NT = 64 * NBW;
  const int64_t n_tiles = (N + NT - 1) / NT;
  const int64_t max_tiles = ((M + MT - 1) / MT + e_local) * n_tiles;
  const int64_t grid = (max_tiles + 7) / 8 * 8;
  DWM_UNSUPPORTED_IF(grid > (1ll << 31) - 1, "gmm_fp4: too many tiles (%lld)", (long long)grid);
  hipLaunchKernelGGL((gmm_fp4_bf16_kernel<MB, NBW, DEPTH>), dim3((unsigned)grid), dim3(kGmmThreads), 0, st,
                     lhs, M, (int)K, w, s, gs, ng, go, e_local, (int)N, out, out_f32);
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
  DWM_UNSUPPORTED_IF(K % 128 != 0 || N % 16 != 0, "gmm_fp4: K %% 128 == 0 and N %% 16 == 0 required");
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
  // 96-row x 256-column tiles, one-step weight prefetch: 240 VGPRs and 60 KB
  // of LDS keep two blocks (8 waves) per CU, measured fastest on the decode
  // and prefill workloads among the (rows, columns, depth) variants tried.
  return launch_gmm<6, 4, 1>(lhs, M, K, weight, scale, group_sizes, num_groups, group_offset, E_local, N,
                             out, out_f32, st);
}
