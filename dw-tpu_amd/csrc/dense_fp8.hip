// Dense FP8 block-quantised GEMM on gfx950.
//
// W8A16 -- the reference dense_fp8.matmul "native" semantics
// (kernels/tpu_inference/kernels/experimental/dense_fp8.py:23-59): for each
// 128-row K block kb, part = dot(x_bf16[:, kb], w_e4m3[kb, :]) in f32, then
// acc += part * s[kb, n] (f32), stored as bf16.
// W8A8 -- e4m3 activations with per-(token, 128-K) f32 scales sx and e4m3
// weights with 128x128 block f32 scales sw:
// acc += part * (sx[m, kb] * sw[kb, n / 128]).
//
// Kernels:
// - M > 16, N % 128 == 0: dense_fp8_mfma_kernel.  W8A16 decodes e4m3 -> bf16
//   (exact: 3 mantissa bits, exponents inside bf16's range) for bf16 MFMA
//   32x32x16; W8A8 runs the fp8 MFMA 32x32x64 on the codes.
// - M <= 16: dense_fp8_skinny_kernel (see below).
// - Other shapes: dense_fp8_kernel, bf16 MFMA 16x16x32 on decoded codes.
// Every product is the exact fp8 (or bf16 x fp8) product; the 128-K partial
// is an f32 sum of them.
//
// Prepacked weight layout (load time, dwm_dense_fp8_prepack):
//   w[(nb * K/128 + kb) * 2048 + lane * 32 + j], lane = 16*q + c,
//   byte j = e4m3 code of k = 128*kb + 32*q + j, column n = 16*nb + c.
// A wave streams one contiguous 2 KiB chunk per (16 columns, 128 K) with two
// 16 B loads per lane; lane (c, q) holds 32 consecutive K of one column, the
// MFMA 16x16x32 B-operand order (8 K per step, 4 steps).
//
// M <= 16: dense_fp8_skinny_kernel (waves split K inside one block, partial
// sums added in LDS in wave order).  Larger M with few tiles: the K loop is
// split over `ksplit` blocks per tile; each writes an f32 partial [ks][M][N]
// to the workspace and dense_fp8_reduce_kernel sums the splits in order and
// rounds once (deterministic).
#include "common.h"

namespace dwm {

constexpr int kDenseThreads = 256;
constexpr int kDLdsRow = 136;  // bf16 per LDS row: 128 + 8 pad

// Two e4m3 codes (bytes 0,1 or 2,3 of src) -> packed bf16x2, exact.
template <bool HI>
__device__ __forceinline__ uint32_t cvt_fp8x2_bf16(uint32_t src) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(src, 1.0f, HI));
}

__global__ void dense_fp8_prepack_kernel(const uint8_t *w, int64_t K, int64_t N, uint8_t *out) {
  // one thread per (nb, kb, lane): 32 bytes
  const int64_t KB = K / 128, N16 = N / 16;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N16 * KB * 64) return;
  const int lane = (int)(t & 63);
  const int64_t r = t >> 6;
  const int64_t kb = r % KB, nb = r / KB;
  const int q = lane >> 4, c = lane & 15;
  const int64_t n = nb * 16 + c;
  uint32_t words[8];
#pragma unroll
  for (int wd = 0; wd < 8; ++wd) {
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = kb * 128 + 32 * q + 4 * wd + i;
      v |= (uint32_t)w[k * N + n] << (8 * i);
    }
    words[wd] = v;
  }
  u32x4_t *dst = (u32x4_t *)(out + (nb * KB + kb) * 2048 + lane * 32);
  dst[0] = u32x4_t{words[0], words[1], words[2], words[3]};
  dst[1] = u32x4_t{words[4], words[5], words[6], words[7]};
}

// A packed pair of bf16 values, each multiplied by `s` (a bf16 value held
// in f32) and rounded to bf16 (round to nearest even): the bf16 x bf16
// product of the reference's "pre" mode (dense_fp8.py:39-43).  The f32
// product of two bf16 values is exact, so this is the correctly rounded
// bf16 product.
__device__ __forceinline__ uint32_t scale_bf16x2(uint32_t v, float s) {
  const float lo = bf16_bits_to_f32(v & 0xFFFFu) * s;
  const float hi = __builtin_bit_cast(float, v & 0xFFFF0000u) * s;
  return f32x2_to_bf16x2_bits(lo, hi);
}

// A8: activations are e4m3 codes with scales sx [M, K/128]; else bf16.
// PRE (W8A16 only): the reference's "pre" rounding -- every weight times the
// bf16-rounded scale of its (K block, column), rounded to bf16, feeds the
// MFMA, and the partials are summed with no scale after the dot.
template <int MB, int NBW, bool A8, bool PRE = false>
__global__ __launch_bounds__(kDenseThreads) void dense_fp8_kernel(
    const void *__restrict__ xin, const float *__restrict__ sx, int64_t M, int K, int N,
    const uint8_t *__restrict__ wpk, const float *__restrict__ sw, int sw_ld, int ksplit,
    uint16_t *__restrict__ out, float *__restrict__ partial) {
  constexpr int MT = 16 * MB;
  __shared__ __attribute__((aligned(16))) uint16_t s_a[2][MT * kDLdsRow];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int KB = K >> 7, N16 = N >> 4;
  const int64_t row0 = (int64_t)blockIdx.y * MT;
  const int rows = (int)min((int64_t)MT, M - row0);
  const int act_mb = (rows + 15) >> 4;
  const int ks = blockIdx.z;
  const int kb_per = (KB + ksplit - 1) / ksplit;
  const int kb_begin = ks * kb_per;
  const int kb_end = min(KB, kb_begin + kb_per);
  const int nb0 = blockIdx.x * (NBW * 4) + wave * NBW;

  const uint8_t *wp[NBW];
  bool nvalid[NBW];
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    nvalid[j] = nb0 + j < N16;
    wp[j] = wpk + (int64_t)(nvalid[j] ? nb0 + j : 0) * KB * 2048 + lane * 32;
  }
  f32x4_t acc[MB][NBW];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[mb][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // lhs staging: 16 rows per i, 16 chunks of 8 bf16 per row (A8: 16 chunks
  // of 8 e4m3 bytes, widened to bf16 on the way into LDS).
  const int srow = tid >> 4, scol = (tid & 15) * 8;
  u32x4_t areg[MB];
  uint32_t areg8[MB][2];
  auto load_a = [&](int kb) {
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      if (i < act_mb) {
        int64_t grow = row0 + 16 * i + srow;
        if (grow >= M) grow = M - 1;
        if (A8) {
          const uint32_t *p = (const uint32_t *)((const uint8_t *)xin + grow * K + (int64_t)kb * 128 + scol);
          areg8[i][0] = p[0];
          areg8[i][1] = p[1];
        } else {
          areg[i] = *(const u32x4_t *)((const uint16_t *)xin + grow * K + (int64_t)kb * 128 + scol);
        }
      }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      if (i < act_mb) {
        u32x4_t v;
        if (A8) {
          v[0] = cvt_fp8x2_bf16<false>(areg8[i][0]);
          v[1] = cvt_fp8x2_bf16<true>(areg8[i][0]);
          v[2] = cvt_fp8x2_bf16<false>(areg8[i][1]);
          v[3] = cvt_fp8x2_bf16<true>(areg8[i][1]);
        } else {
          v = areg[i];
        }
        *(u32x4_t *)(&s_a[buf][(16 * i + srow) * kDLdsRow + scol]) = v;
      }
    }
  };

  u32x4_t wlo[NBW], whi[NBW], nlo[NBW], nhi[NBW];
  if (kb_begin < kb_end) {
    load_a(kb_begin);
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const u32x4_t *p = (const u32x4_t *)(wp[j] + (int64_t)kb_begin * 2048);
      wlo[j] = p[0];
      whi[j] = p[1];
    }
    store_a(0);
  }
  __syncthreads();

  const int arow = lane & 15, acol = 32 * (lane >> 4), qrow = 4 * (lane >> 4);
  for (int kb = kb_begin; kb < kb_end; ++kb) {
    const int buf = (kb - kb_begin) & 1;
    const bool more = kb + 1 < kb_end;
    if (more) {
      load_a(kb + 1);
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        const u32x4_t *p = (const u32x4_t *)(wp[j] + (int64_t)(kb + 1) * 2048);
        nlo[j] = p[0];
        nhi[j] = p[1];
      }
    }
    f32x4_t part[MB][NBW];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < NBW; ++j) part[mb][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const uint16_t *abase = &s_a[buf][arow * kDLdsRow + acol];
    // PRE: the bf16-rounded scale of each of the lane's weight columns.
    float pscale[NBW];
    if constexpr (PRE) {
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        const int64_t col = (int64_t)(nvalid[j] ? nb0 + j : 0) * 16 + (lane & 15);
        pscale[j] = bf16_bits_to_f32(f32_to_bf16_bits(sw[(int64_t)kb * sw_ld + col]));
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4_t bfrag[NBW];
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        // 8 e4m3 codes of this step: words 2s, 2s+1 of the lane's 32 bytes
        const uint32_t w0 = s < 2 ? wlo[j][2 * s] : whi[j][2 * s - 4];
        const uint32_t w1 = s < 2 ? wlo[j][2 * s + 1] : whi[j][2 * s - 3];
        bfrag[j][0] = cvt_fp8x2_bf16<false>(w0);
        bfrag[j][1] = cvt_fp8x2_bf16<true>(w0);
        bfrag[j][2] = cvt_fp8x2_bf16<false>(w1);
        bfrag[j][3] = cvt_fp8x2_bf16<true>(w1);
        if constexpr (PRE) {
#pragma unroll
          for (int i = 0; i < 4; ++i) bfrag[j][i] = scale_bf16x2(bfrag[j][i], pscale[j]);
        }
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        if (mb < act_mb) {
          const u32x4_t a = *(const u32x4_t *)(abase + mb * 16 * kDLdsRow + 8 * s);
#pragma unroll
          for (int j = 0; j < NBW; ++j)
            part[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, bfrag[j]), part[mb][j], 0, 0, 0);
        }
      }
    }
    // acc += part * scale (f32 multiply, then f32 add); PRE: acc += part
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int64_t col = (int64_t)(nvalid[j] ? nb0 + j : 0) * 16 + (lane & 15);
      const float wscale = PRE ? 1.0f : (A8 ? sw[(int64_t)kb * sw_ld + (col >> 7)] : sw[(int64_t)kb * sw_ld + col]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        if (mb < act_mb) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float f = wscale;
            if (A8) {
              int64_t m = row0 + mb * 16 + qrow + r;
              if (m >= M) m = M - 1;
              f = sx[m * KB + kb] * wscale;
            }
            acc[mb][j][r] = acc[mb][j][r] + part[mb][j][r] * f;
          }
        }
      }
    }
    if (more) {
      store_a(buf ^ 1);
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        wlo[j] = nlo[j];
        whi[j] = nhi[j];
      }
    }
    __syncthreads();
  }

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
          if (partial) partial[(int64_t)ks * M * N + o] = acc[mb][j][r];
          else out[o] = f32_to_bf16_bits(acc[mb][j][r]);
        }
      }
    }
  }
}

// Skinny M (<= 16 rows, decode): one block owns 16 columns and KS waves split
// its K steps.  Each wave streams its contiguous prepacked weight chunks and
// its lhs fragments (straight from L2, only rows < M) through a D-deep
// register ring; there is no LDS staging and no barrier in the K loop.
// The waves' f32 partial sums are added in LDS in wave order (deterministic)
// and rounded once, in the same launch.
template <int KS, int D, bool A8>
__global__ __launch_bounds__(64 * KS) void dense_fp8_skinny_kernel(
    const void *__restrict__ xin, const float *__restrict__ sx, int M, int K, int N,
    const uint8_t *__restrict__ wpk, const float *__restrict__ sw, int sw_ld, uint16_t *__restrict__ out) {
  __shared__ f32x4_t s_red[KS - 1][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int KB = K >> 7;
  const int nb = blockIdx.x;
  const int kb_per = (KB + KS - 1) / KS;
  const int kb_begin = wave * kb_per;
  const int kb_end = min(KB, kb_begin + kb_per);
  const int r = lane & 15, q = lane >> 4;
  const bool rok = r < M;
  const int64_t col = (int64_t)nb * 16 + r;  // C layout: column lane % 16, rows 4 q .. 4 q + 3
  const uint8_t *const wp = wpk + (int64_t)nb * KB * 2048 + lane * 32;
  // lhs fragment of MFMA step s: row r, k = 128 kb + 32 q + 8 s .. + 7
  const uint8_t *const xrow = (const uint8_t *)xin + (int64_t)(rok ? r : 0) * K * (A8 ? 1 : 2) + 32 * q * (A8 ? 1 : 2);
  // Everything a K block reads -- its weight chunk, its lhs fragments and its
  // scales -- travels in one D-deep register ring, loaded in K-block order:
  // the wait for block kb then covers only loads issued before those of
  // block kb + 1 (vector loads complete in order), so D blocks stay in flight.
  constexpr int XW = A8 ? 2 : 4;  // 16-byte lhs loads per K block
  u32x4_t wlo[D], whi[D], xa[D][XW];
  float wsc[D], xsc[D][4];
  auto load = [&](int slot, int kb) {
    const u32x4_t *p = (const u32x4_t *)(wp + (int64_t)kb * 2048);
    wlo[slot] = p[0];
    whi[slot] = p[1];
    if (rok) {
      const u32x4_t *xp = (const u32x4_t *)(xrow + (int64_t)kb * (A8 ? 128 : 256));
#pragma unroll
      for (int s = 0; s < XW; ++s) xa[slot][s] = xp[s];
    } else {
#pragma unroll
      for (int s = 0; s < XW; ++s) xa[slot][s] = u32x4_t{0u, 0u, 0u, 0u};
    }
    wsc[slot] = A8 ? sw[(int64_t)kb * sw_ld + (col >> 7)] : sw[(int64_t)kb * sw_ld + col];
    if (A8) {
#pragma unroll
      for (int i = 0; i < 4; ++i) xsc[slot][i] = sx[(int64_t)min(4 * q + i, M - 1) * KB + kb];
    }
  };
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (kb_begin + d < kb_end) load(d, kb_begin + d);
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int kb0 = kb_begin; kb0 < kb_end; kb0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int kb = kb0 + d;
      if (kb >= kb_end) break;
      u32x4_t a[4];
      if (A8) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint32_t w0 = s < 2 ? xa[d][0][2 * s] : xa[d][1][2 * s - 4];
          const uint32_t w1 = s < 2 ? xa[d][0][2 * s + 1] : xa[d][1][2 * s - 3];
          a[s] = u32x4_t{cvt_fp8x2_bf16<false>(w0), cvt_fp8x2_bf16<true>(w0), cvt_fp8x2_bf16<false>(w1),
                         cvt_fp8x2_bf16<true>(w1)};
        }
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) a[s] = xa[d][s];
      }
      const u32x4_t lo = wlo[d], hi = whi[d];
      const float wscale = wsc[d];
      float f[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) f[i] = A8 ? xsc[d][i] * wscale : wscale;
      if (kb + D < kb_end) load(d, kb + D);
      f32x4_t part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t w0 = s < 2 ? lo[2 * s] : hi[2 * s - 4];
        const uint32_t w1 = s < 2 ? lo[2 * s + 1] : hi[2 * s - 3];
        const u32x4_t b = {cvt_fp8x2_bf16<false>(w0), cvt_fp8x2_bf16<true>(w0), cvt_fp8x2_bf16<false>(w1),
                           cvt_fp8x2_bf16<true>(w1)};
        part = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a[s]),
                                                       __builtin_bit_cast(bf16x8_t, b), part, 0, 0, 0);
      }
      // acc += part * scale (f32 multiply, then f32 add)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = acc[i] + part[i] * f[i];
    }
  }
  if (wave > 0) s_red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int w = 0; w < KS - 1; ++w) acc = acc + s_red[w][lane];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * q + i;
    if (m < M) out[(int64_t)m * N + col] = f32_to_bf16_bits(acc[i]);
  }
}

// ---------------------------------------------------------------------------
// Large M: block tiles of BM x BN = (64 WM) x (32 JN WN), each wave a
// 64 x 32 JN output of 2 x JN MFMA 32x32 tiles (JN = 2; the 128-row W8A16
// tiles run 8 waves of JN = 1, two waves per SIMD, one hiding the other's
// LDS reads and conversions: 3-8% faster than 4 waves of 64 x 64 at
// M = 128 .. 1024, the same bits).  All waves stream 64-deep K steps of the
// lhs tile, the prepacked weight chunks and the step's scales into a ring of
// NS LDS stages with direct global -> LDS loads (the only vector-memory
// operations in the loop, so the waits are exact counts), one barrier per
// step.  W8A16 decodes the e4m3 weights to bf16 (exact) and runs bf16 MFMA
// 32x32x16, 64 K per step; W8A8 runs the fp8 MFMA 32x32x64 on the codes, a
// whole 128-deep K block per step.  Each K block's partial sum is scaled once
// into the f32 accumulator (acc = fma(part, scale, acc)).
//
// Stage layout: lhs rows of 128 bytes (64 K of bf16, or 128 K of e4m3: every
// lhs load takes whole 128-byte lines), their 16-byte chunks swizzled (chunk
// c of row r at c ^ ((r >> 1) & 7)) so that a fragment read by 16 lanes of
// consecutive rows hits distinct bank groups; then per 16 columns the 1 KiB
// halves of the prepacked 2 KiB chunk that the step covers (W8A16 one, W8A8
// both; in a half, 16-byte slot 32 q + 2 c + p holds k = 32 q + 16 p .. + 15
// of column c), stored with p flipped for c >= 8 (lane l loads slot
// l ^ ((l >> 4) & 1)), so that 16 lanes reading one slot of 16 consecutive
// columns hit distinct bank groups; then the scales: W8A16 the block's
// column scales of the step's K block, W8A8 sw[kb, n0/128] (every wave loads
// it, so each wave issues the same loads per step).  W8A8's row scales sit
// outside the ring: every SX_KB K blocks the waves load sx[row0 .. + BM - 1,
// the next SX_KB K blocks] into one of two [BM][SX_KB] f32 buffers, rows of
// 4 * SX_KB contiguous bytes (a column of sx read per step would touch one
// line per row).
template <int WM, int WN, bool A8, int JN = 2>
struct DenseMfmaCfg {
  static constexpr int WAVES = WM * WN, THREADS = 64 * WAVES, WCOLS = WN, JCOLS = JN;
  static constexpr int BM = 64 * WM, BN = 32 * JN * WN;
  static constexpr int A_ROW = 128;            // lhs bytes per row per step: 64 K of bf16 or 128 K of e4m3
  static constexpr int W_STEP = A8 ? 2048 : 1024;  // weight bytes per 16 columns per step
  static constexpr int A = 0;
  static constexpr int B = BM * A_ROW;
  static constexpr int S = B + BN / 16 * W_STEP;
  static constexpr int S_BYTES = WAVES * 256;  // one 64-value scale load per wave
  static constexpr int STAGE = (S + S_BYTES + 1023) / 1024 * 1024;
  static constexpr int SX_KB = BM == 256 ? 4 : 8;                  // W8A8: K blocks per row-scale chunk
  static constexpr int SX_BUF = BM * SX_KB * 4;                    // [BM rows][SX_KB] f32
  static constexpr int SX_BYTES = A8 ? 2 * SX_BUF : 0;
  static constexpr int SX_LOADS = A8 ? SX_BUF / 256 / WAVES : 0;   // 256-byte loads per wave per chunk
  static constexpr int A_LOADS = BM * A_ROW / 1024 / WAVES;        // 1 KiB lhs loads per wave per step
  static constexpr int B_LOADS = BN / 16 * W_STEP / 1024 / WAVES;  // 1 KiB weight loads per wave per step
  static constexpr int S_LOADS = 1;                                // 256-byte scale loads per wave per step
  static constexpr int LOADS = A_LOADS + B_LOADS + S_LOADS;
  static_assert(A_LOADS * WAVES * 1024 == BM * A_ROW && B_LOADS * WAVES * 1024 == BN / 16 * W_STEP,
                "loads split over the waves");
  static_assert(!A8 || (SX_LOADS * WAVES * 256 == SX_BUF && WAVES % 2 == 0), "row-scale loads split over the waves");
  static_assert(BN == 128, "one 128-column weight-scale block per tile");
  static_assert(!A8 || JN == 2, "W8A8 waves own two 32-column tiles");
};

typedef __attribute__((ext_vector_type(8))) int i32x8_t;

// Per-wave step accounting of dense_fp8_mfma_kernel, compiled into the
// library's timeline build only (-DDWTPU_TIMELINE, libdwtpu_moe_timeline.so;
// the product library has no trace of it).  Every wave sums its shader
// cycles (s_memtime) by phase and lane 0 stores kDsSlots words for wave w of
// block b (linear block index) at (16 b + w) * kDsSlots: 0 prologue (entry to
// the first wait), 1 waits for data, 2 barriers, 3 work between barriers,
// 4 epilogue (loop end to its stores complete), 5 steps, 6 HW_ID | XCC_ID << 32,
// 7 and 8 s_memrealtime (100 MHz) at entry and exit, 9 s_memtime from entry
// to exit.
[[maybe_unused]] constexpr int kDsSlots = 10;
#ifdef DWTPU_TIMELINE
static __device__ uint64_t *g_dense_steps;
static __device__ int64_t g_dense_steps_waves;
#define DWM_DS(...) __VA_ARGS__
#else
#define DWM_DS(...)
#endif

template <class C, bool A8, int NS, bool PF = false>
__global__ __launch_bounds__(C::THREADS) void dense_fp8_mfma_kernel(
    const void *__restrict__ xin, const float *__restrict__ sx, int64_t M, int K, int N,
    const uint8_t *__restrict__ wpk, const float *__restrict__ sw, int sw_ld, int ksplit, uint16_t *__restrict__ out,
    float *__restrict__ partial) {
  __shared__ __attribute__((aligned(1024))) uint8_t s_lds[NS * C::STAGE + C::SX_BYTES];
  DWM_DS(const uint64_t ds_rt0 = __builtin_amdgcn_s_memrealtime(); const uint64_t ds_t0 = __builtin_amdgcn_s_memtime();
         uint64_t ds_prev = ds_t0, ds_pro = 0, ds_wait = 0, ds_bar = 0, ds_work = 0; int ds_n = 0;)
  // The wave index is made wave-uniform, so that every load address below
  // is a scalar base plus a per-lane 32-bit offset (no per-step vector
  // address arithmetic) and the LDS destinations are scalar.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c32 = lane & 31, h = lane >> 5;
  const int KB = K >> 7, N16 = N >> 4;
  // Split K: blocks z = 0 .. ksplit-1 take consecutive runs of K blocks.
  const int kb_per = (KB + ksplit - 1) / ksplit;
  const int kb0 = blockIdx.z * kb_per;
  const int nkb = max(0, min(KB, kb0 + kb_per) - kb0);
  const int T = A8 ? nkb : 2 * nkb;  // steps of this block (W8A8 128 K deep, W8A16 64 K)
  const int64_t row0 = (int64_t)blockIdx.y * C::BM;
  const int n0 = blockIdx.x * C::BN;
  const int wm = wave / C::WCOLS, wn = wave % C::WCOLS;
  // ---- load addressing (per lane, per step t) ----
  // lhs: load i of this wave covers rows 8 (wave + WAVES i) .. + 7; lane l
  // fills physical chunk l % 8 of row + l / 8 with the logical chunk of the
  // swizzle.
  uint32_t aoff[C::A_LOADS];
#pragma unroll
  for (int i = 0; i < C::A_LOADS; ++i) {
    const int r = 8 * (wave + C::WAVES * i) + (lane >> 3);
    int64_t gr = row0 + r;
    if (gr >= M) gr = M - 1;
    const int lc = (lane & 7) ^ ((r >> 1) & 7);
    aoff[i] = (uint32_t)(gr * (int64_t)K * (A8 ? 1 : 2)) + (uint32_t)lc * 16u;
  }
  const __amdgpu_buffer_rsrc_t arsrc = make_rsrc(xin, (uint32_t)(M * K * (A8 ? 1 : 2)));
  const __amdgpu_buffer_rsrc_t wrsrc = make_rsrc(wpk, (uint32_t)((int64_t)K * N));
  // weights: load i of this wave fills 1 KiB slot g = wave + WAVES i of the
  // stage's weight region: W8A16 the step's half of 16-column group g, W8A8
  // half g % 2 of group g / 2.
  uint32_t woff[C::B_LOADS];
#pragma unroll
  for (int i = 0; i < C::B_LOADS; ++i) {
    const int g = wave + C::WAVES * i;
    int nb = n0 / 16 + (A8 ? g >> 1 : g);
    if (nb >= N16) nb = N16 - 1;
    woff[i] = (uint32_t)nb * (uint32_t)KB * 2048u + (A8 ? (uint32_t)(g & 1) * 1024u : 0u) +
              (uint32_t)(lane ^ ((lane >> 4) & 1)) * 16u;
  }
  // scales: W8A16 wave w loads columns n0 + 64 w + lane of sw[kb]; W8A8
  // every wave loads sw[kb, n0/128] (all lanes the one value).
  const __amdgpu_buffer_rsrc_t srsrc = make_rsrc(sw, (uint32_t)KB * (uint32_t)sw_ld * 4u);
  const uint32_t slane = A8 ? (uint32_t)(n0 / 128) * 4u : (uint32_t)min(n0 + 64 * wave + lane, N - 1) * 4u;
  const uint32_t sstride = (uint32_t)sw_ld * 4u;  // bytes per K block
  // W8A8 row scales: load i of this wave covers block rows XR (wave + WAVES i)
  // .. + XR - 1 (XR = 64 / SX_KB), lane l row + l / SX_KB, K block
  // kb0 + SX_KB c + l % SX_KB of chunk c (rows past M repeat the last row; K
  // blocks past the block's run are never read).
  constexpr int XR = 64 / C::SX_KB;
  __amdgpu_buffer_rsrc_t xrsrc;
  uint32_t xoff[C::SX_LOADS > 0 ? C::SX_LOADS : 1];
  if constexpr (A8) {
    xrsrc = make_rsrc(sx, (uint32_t)(M * KB * 4));
#pragma unroll
    for (int i = 0; i < C::SX_LOADS; ++i) {
      int64_t r = row0 + XR * (wave + C::WAVES * i) + lane / C::SX_KB;
      if (r >= M) r = M - 1;
      xoff[i] = (uint32_t)(r * KB) * 4u + (uint32_t)(lane % C::SX_KB) * 4u;
    }
  }
  uint8_t *const s_sx = s_lds + NS * C::STAGE;
  auto issue_sx = [&](int c) {  // row scales of K blocks kb0 + SX_KB c .. into buffer c % 2
#pragma unroll
    for (int i = 0; i < C::SX_LOADS; ++i)
      buffer_load_lds(4, xrsrc, s_sx + (c & 1) * C::SX_BUF + (wave + C::WAVES * i) * 256, xoff[i],
                      (uint32_t)(kb0 + C::SX_KB * c) * 4u);
  };
  auto issue = [&](int stage, int t) {
    uint8_t *const st = s_lds + stage * C::STAGE;
    const uint32_t kb = (uint32_t)(kb0 + (A8 ? t : t >> 1));
    const uint32_t wstep = A8 ? kb * 2048u : kb * 2048u + (uint32_t)(t & 1) * 1024u;
    const uint32_t astep = (uint32_t)((A8 ? kb0 : kb0 * 2) + t) * 128u;  // lhs bytes before the step
#pragma unroll
    for (int i = 0; i < C::A_LOADS; ++i)
      buffer_load_lds(16, arsrc, st + C::A + (wave + C::WAVES * i) * 1024, aoff[i], astep);
#pragma unroll
    for (int i = 0; i < C::B_LOADS; ++i)
      buffer_load_lds(16, wrsrc, st + C::B + (wave + C::WAVES * i) * 1024, woff[i], wstep);
    buffer_load_lds(4, srsrc, st + C::S + wave * 256, slane, kb * sstride);
  };
  // ---- compute addressing ----
  const int rA[2] = {64 * wm + c32, 64 * wm + 32 + c32};    // block-local rows of the 2 row tiles
  constexpr int JN = C::JCOLS;
  int cB[JN];  // block-local columns of the wave's JN 32-column tiles
#pragma unroll
  for (int j = 0; j < JN; ++j) cB[j] = 32 * JN * wn + 32 * j + c32;
  f32x16_t acc[2][JN], part[2][JN];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < JN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  // PF: a wave reads the fragments of MFMA substep s + 1 (of step t + 1
  // after the last substep of step t) while substep s's MFMAs run, so the
  // barrier of step t also waits for step t + 1 to land.
  constexpr int PENDING = C::LOADS * (NS - (PF ? 3 : 2));
  static_assert(PENDING >= 0 && PENDING < 64, "vmcnt range");
  static_assert(!A8 || (PF && NS - 1 <= C::SX_KB), "W8A8 prefetches its fragments; row-scale chunk timing");
  // W8A8: row-scale chunk c + 1 is issued before step SX_KB c's refill, so
  // it is older than the loads of every step from SX_KB (c + 1) on (issued
  // at step SX_KB (c + 1) - NS + 1 or later) and the wait for such a step
  // covers it; the buffer it fills was last read in the fold of step
  // SX_KB c - 1.
  if (T > 0) {
    if constexpr (A8) issue_sx(0);
#pragma unroll
    for (int t = 0; t < NS - 1; ++t) issue(t, min(t, T - 1));
  }
  // W8A16: lane (c32, h) takes k = 32 h + 8 ks .. + 7 of the step in MFMA
  // substep ks (the same k for the lhs chunk and the weight codes, so every
  // product is formed once): per step 32 codes of each of its 2 columns, per
  // substep one lhs chunk of each of its 2 rows.
  struct Frag16 {
    u32x4_t a[2];
  };
  u32x4_t w16[JN][2];  // [column tile][k 32 h .. + 15, + 16 .. + 31]
  auto read16w = [&](const uint8_t *st, u32x4_t (*w)[2]) {
#pragma unroll
    for (int j = 0; j < JN; ++j) {
      const int c = cB[j] & 15;
      const uint8_t *pw = st + C::B + (cB[j] >> 4) * 1024 + (32 * h + 2 * c) * 16;
      w[j][0] = *(const u32x4_t *)(pw + 16 * (c >> 3));
      w[j][1] = *(const u32x4_t *)(pw + 16 * ((c >> 3) ^ 1));
    }
  };
  auto read16 = [&](const uint8_t *st, int ks, Frag16 &f) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = rA[i];
      const int pc = (4 * h + ks) ^ ((r >> 1) & 7);
      f.a[i] = *(const u32x4_t *)(st + C::A + r * 128 + pc * 16);
    }
  };
  auto mma16 = [&](const Frag16 &f, const u32x4_t (*w)[2], int ks, bool first) {
    u32x4_t b[JN];
#pragma unroll
    for (int j = 0; j < JN; ++j) {
      const uint32_t w0 = w[j][ks >> 1][2 * (ks & 1)], w1 = w[j][ks >> 1][2 * (ks & 1) + 1];
      b[j][0] = cvt_fp8x2_bf16<false>(w0);
      b[j][1] = cvt_fp8x2_bf16<true>(w0);
      b[j][2] = cvt_fp8x2_bf16<false>(w1);
      b[j][3] = cvt_fp8x2_bf16<true>(w1);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        const f32x16_t z = {};
        part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f.a[i]),
                                                             __builtin_bit_cast(bf16x8_t, b[j]),
                                                             first ? z : part[i][j], 0, 0, 0);
      }
  };
  // W8A8 step (64 deep): 32 lhs codes per row tile and 32 weight codes per
  // column tile.
  struct Frag8 {
    i32x8_t a[2], b[2];
  };
  auto read8 = [&](const uint8_t *st, int hs, Frag8 &f) {  // substep hs: k = 64 hs .. + 63 of the step
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = rA[i];
      const u32x4_t lo = *(const u32x4_t *)(st + C::A + r * 128 + (((4 * hs + h) ^ ((r >> 1) & 7)) * 16));
      const u32x4_t hi = *(const u32x4_t *)(st + C::A + r * 128 + (((4 * hs + 2 + h) ^ ((r >> 1) & 7)) * 16));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f.a[i][q] = (int)lo[q];
        f.a[i][4 + q] = (int)hi[q];
      }
    }
#pragma unroll
    for (int j = 0; j < JN; ++j) {
      const int col = cB[j];
      const int c = col & 15;
      const uint8_t *pc = st + C::B + (col >> 4) * 2048 + hs * 1024 + c * 32 + 16 * (h ^ (c >> 3));
      const u32x4_t lo = *(const u32x4_t *)pc;
      const u32x4_t hi = *(const u32x4_t *)(pc + 16 * 32);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f.b[j][q] = (int)lo[q];
        f.b[j][4 + q] = (int)hi[q];
      }
    }
  };
  auto mma8 = [&](const Frag8 &f, bool first) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        const f32x16_t z = {};
        part[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[i], f.b[j], first ? z : part[i][j], 0, 0, 0,
                                                                     127, 0, 127);
      }
  };
  Frag16 f16;
  u32x4_t w16n[JN][2];  // PF: the next step's weight codes
  Frag8 f8;
  // W8A16: pairs of 64-deep steps (t, t + 1), a K block per pair; W8A8: one
  // step per K block.
  // W8A16 runs the loop in copies of NS steps, so that the stage of every
  // step (cur = step % NS) is known in its copy and every stage address is a
  // constant offset (a third fewer VALU instructions per MFMA).  W8A8 keeps
  // one copy: with NS of them its 256-row variant spills.
  constexpr int TS = A8 ? 1 : 2;
  constexpr int REPS = A8 ? 1 : NS;
  int cur_rt = 0;  // W8A8: the stage of step t
  for (int t0 = 0; t0 < T; t0 += TS * REPS) {
#pragma unroll
  for (int rep = 0; rep < REPS; ++rep) {
    const int t = t0 + rep * TS;
    if (t >= T) break;
#pragma unroll
    for (int hs = 0; hs < TS; ++hs) {
      const int cur = A8 ? cur_rt : (rep * TS + hs) % NS;
      DWM_DS(const uint64_t ds_ta = __builtin_amdgcn_s_memtime();)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(PENDING));
      DWM_DS(const uint64_t ds_tb = __builtin_amdgcn_s_memtime();)
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      DWM_DS(const uint64_t ds_tc = __builtin_amdgcn_s_memtime();
             if (ds_n == 0) ds_pro = ds_ta - ds_prev; else ds_work += ds_ta - ds_prev;
             ds_wait += ds_tb - ds_ta; ds_bar += ds_tc - ds_tb; ds_prev = ds_tc; ++ds_n;)
      // Every wave is done with step t + hs - 1: refill its stage.
      if constexpr (A8) {
        if (t % C::SX_KB == 0 && t + C::SX_KB < T) issue_sx(t / C::SX_KB + 1);
      }
      issue(cur == 0 ? NS - 1 : cur - 1, min(t + hs + NS - 1, T - 1));
      const uint8_t *const st = s_lds + cur * C::STAGE;
      const int nxt = cur == NS - 1 ? 0 : cur + 1;
      // PF: step t + hs + 1 has landed and its stage is not refilled before
      // the next barrier (in the last step the prefetch reads stale stage
      // contents that are never used).
      const uint8_t *const sx = s_lds + nxt * C::STAGE;
      if constexpr (!A8) {
        if constexpr (PF) {
          if (t + hs == 0) {
            read16w(st, w16n);
            read16(st, 0, f16);
          }
#pragma unroll
          for (int j = 0; j < JN; ++j) {
            w16[j][0] = w16n[j][0];
            w16[j][1] = w16n[j][1];
          }
        } else {
          read16w(st, w16);
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          if constexpr (PF) {
            const Frag16 c = f16;
            __builtin_amdgcn_sched_barrier(0);
            if (ks < 3) read16(st, ks + 1, f16);
            else read16(sx, 0, f16);
            if (ks == 0) read16w(sx, w16n);
            mma16(c, w16, ks, hs == 0 && ks == 0);
            __builtin_amdgcn_sched_barrier(0);
          } else {
            read16(st, ks, f16);
            mma16(f16, w16, ks, hs == 0 && ks == 0);
          }
        }
      } else {
        // Two 64-deep substeps; each reads the next one's fragments (after
        // the second, the next step's first) during its MFMAs.
        if (t == 0) read8(st, 0, f8);
        {
          const Frag8 c = f8;
          __builtin_amdgcn_sched_barrier(0);
          read8(st, 1, f8);
          mma8(c, true);
          __builtin_amdgcn_sched_barrier(0);
        }
        {
          const Frag8 c = f8;
          __builtin_amdgcn_sched_barrier(0);
          read8(sx, 0, f8);
          mma8(c, false);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (A8 || hs == 1) {
        // The K block is complete: acc += part * scale.
        if constexpr (!A8) {
#pragma unroll
          for (int j = 0; j < JN; ++j) {
            const float sc = *(const float *)(st + C::S + cB[j] * 4);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
              for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(part[i][j][r], sc, acc[i][j][r]);
          }
        } else {
          const float swv = *(const float *)(st + C::S);
          // sx[row, kb0 + t] of block row r at s_sx[t / SX_KB % 2][r][t % SX_KB]
          const float *const xs = (const float *)(s_sx + ((t / C::SX_KB) & 1) * C::SX_BUF) + t % C::SX_KB;
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            float f[16];
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
              for (int q = 0; q < 4; ++q) f[4 * g + q] = xs[(rA[i] - c32 + 8 * g + 4 * h + q) * C::SX_KB] * swv;
#pragma unroll
            for (int j = 0; j < JN; ++j)
#pragma unroll
              for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(part[i][j][r], f[r], acc[i][j][r]);
          }
        }
      }
      if constexpr (A8) cur_rt = cur_rt == NS - 1 ? 0 : cur_rt + 1;
    }
  }
  }
  DWM_DS(const uint64_t ds_te = __builtin_amdgcn_s_memtime(); ds_work += ds_te - ds_prev;)
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  // Epilogue: the 32x32 layout (register r of lane (c32, h) is row
  // 8 (r / 4) + 4 h + r % 4, column c32).
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < JN; ++j) {
      const int64_t col = n0 + cB[j];
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = row0 + rA[i] - c32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (row < M) {
          if (partial) partial[((int64_t)blockIdx.z * M + row) * N + col] = acc[i][j][r];
          else out[row * N + col] = f32_to_bf16_bits(acc[i][j][r]);
        }
      }
    }
  }
#ifdef DWTPU_TIMELINE
  __builtin_amdgcn_s_waitcnt(0);
  {
    const uint64_t ds_end = __builtin_amdgcn_s_memtime(), ds_rt1 = __builtin_amdgcn_s_memrealtime();
    const int64_t blk = blockIdx.x + (int64_t)gridDim.x * (blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
    const int64_t slot = blk * 16 + wave;
    if (lane == 0 && g_dense_steps && slot < g_dense_steps_waves) {
      uint64_t *const p = g_dense_steps + slot * kDsSlots;
      p[0] = ds_pro;
      p[1] = ds_wait;
      p[2] = ds_bar;
      p[3] = ds_work;
      p[4] = ds_end - ds_te;
      p[5] = (uint64_t)ds_n;
      p[6] = (uint32_t)__builtin_amdgcn_s_getreg(4 | (31 << 11)) |
             ((uint64_t)(uint32_t)__builtin_amdgcn_s_getreg(20 | (31 << 11)) << 32);
      p[7] = ds_rt0;
      p[8] = ds_rt1;
      p[9] = ds_end - ds_t0;
    }
  }
#endif
}

// out = bf16(sum_{ks} partial[ks]) in split order.  Each thread issues the
// loads of KC runs before it adds them (in order): a wave has KC partial
// loads in flight rather than one round trip per run.
template <int KC>
__global__ void dense_fp8_reduce_kernel(const float *partial, int ksplit, int64_t MN, uint16_t *out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < MN; i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.0f;
    for (int k0 = 0; k0 < ksplit; k0 += KC) {
      float p[KC];
#pragma unroll
      for (int j = 0; j < KC; ++j) p[j] = partial[(int64_t)min(k0 + j, ksplit - 1) * MN + i];
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        if (k0 + j == 0) s = p[0];
        else if (k0 + j < ksplit) s = s + p[j];
      }
    }
    out[i] = f32_to_bf16_bits(s);
  }
}

// The same sum, 4 consecutive outputs per thread (16-byte partial loads,
// 8-byte stores; MN % 4 == 0, partial and out 16-byte aligned).
template <int KC>
__global__ void dense_fp8_reduce4_kernel(const float *__restrict__ partial, int ksplit, int64_t MN,
                                         uint16_t *__restrict__ out) {
  const int64_t n4 = MN >> 2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
    f32x4_t s = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < ksplit; k0 += KC) {
      f32x4_t p[KC];
#pragma unroll
      for (int j = 0; j < KC; ++j) p[j] = ((const f32x4_t *)(partial + (int64_t)min(k0 + j, ksplit - 1) * MN))[i];
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        if (k0 + j == 0) {
          s = p[0];
        } else if (k0 + j < ksplit) {
          s[0] = s[0] + p[j][0];
          s[1] = s[1] + p[j][1];
          s[2] = s[2] + p[j][2];
          s[3] = s[3] + p[j][3];
        }
      }
    }
    u32x2_t o;
    o[0] = f32x2_to_bf16x2_bits(s[0], s[1]);
    o[1] = f32x2_to_bf16x2_bits(s[2], s[3]);
    ((u32x2_t *)out)[i] = o;
  }
}

// ---------------------------------------------------------------------------
// Launch plans.  A dwm_dense_plan names one launch: the kernel family, its
// block tile, the number of K runs that share an output tile (blocks that
// write f32 partials summed in run order by dense_fp8_reduce_kernel, or the
// skinny kernel's waves) and the ring depth.  default_plan() is the library's
// own choice; check_plan() admits exactly the instantiated configurations.

// Tiled kernel (any N % 16 == 0): 16 MB rows x 64 NBW columns.
static dwm_dense_plan tiled_default(int64_t M, int64_t K, int64_t N) {
  dwm_dense_plan p{DWM_DENSE_TILED, 128, 128, 1, 2};
  if (M <= 16) p.tile_m = 16, p.tile_n = 64;
  else if (M <= 64) p.tile_m = 64;
  const int64_t tiles = ((N + p.tile_n - 1) / p.tile_n) * ((M + p.tile_m - 1) / p.tile_m);
  const int64_t KB = K / 128;
  int ks = 1;
  while (tiles * ks < 512 && ks * 2 <= KB && ks < 16) ks *= 2;  // fill the 256 CUs twice over
  p.ksplit = ks;
  return p;
}

// MFMA path (M > 16, N % 128 == 0): W8A16 128x128 tiles (8 waves, two or
// three 25 KB stages: two blocks per CU), 256x128 tiles (8 waves) when those
// alone fill the grid; W8A8 256x128 tiles (8 waves, three 50 KB stages of
// one K block each, fragments read one substep ahead) from M >= 256, 128x128
// below (four 33 KB stages).  K is split over blocks until the grid covers
// the 256 CUs.
static bool dense_mfma_ok(int64_t M, int64_t K, int64_t N, int tile_m) {
  return M > 16 && N % 128 == 0 && M * K * 2 < (1ll << 32) && K * N < (1ll << 32) &&
         (M + tile_m - 1) / tile_m <= 65535;
}

// Smallest run count with the same runs: no run is left empty.
static int whole_runs(int64_t KB, int ks) {
  const int64_t per = (KB + ks - 1) / ks;
  return (int)((KB + per - 1) / per);
}

static dwm_dense_plan default_plan(int64_t M, int64_t K, int64_t N, bool a8) {
  const int64_t KB = K / 128;
  if (dense_mfma_ok(M, K, N, 128)) {
    const int tm = (a8 && M >= 256) ? 256 : 128;
    const int64_t tiles = (N / 128) * ((M + tm - 1) / tm);
    int ks = 1;
    while (tiles * ks < 256 && ks * 2 <= KB && ks < 16) ks *= 2;
    ks = whole_runs(KB, ks);
    if (a8) return {DWM_DENSE_MFMA, tm, 128, ks, tm == 256 ? 3 : 4};
    // Enough rows for 256 x 128 tiles to fill the grid: half the weight
    // re-reads of 128-row tiles (8 waves, one block per CU).
    if (ks == 1 && (N / 128) * ((M + 255) / 256) >= 256) return {DWM_DENSE_MFMA, 256, 128, 1, 2};
    // Two blocks per CU either way; a grid that fits one round takes the
    // deeper ring.
    return {DWM_DENSE_MFMA, 128, 128, ks, tiles * ks <= 512 ? 3 : 2};
  }
  // 16 waves split K, two K blocks (weights, lhs fragments and scales) in
  // flight per wave; 4/8/16 waves x 2..7 blocks in flight all measured
  // within 0.5 us at K=7168, N=4096: the 29 MB stream plus launch and
  // start-up latency sets the time (8 us at M = 1).
  if (M <= 16) return {DWM_DENSE_SKINNY, 16, 16, 16, 2};
  dwm_dense_plan p = tiled_default(M, K, N);
  p.ksplit = whole_runs(KB, p.ksplit);
  return p;
}

static int check_plan(int64_t M, int64_t K, int64_t N, bool a8, const dwm_dense_plan &p) {
  const int64_t KB = K / 128;
  const char *const v = a8 ? "w8a8" : "w8a16";
  if (p.kernel == DWM_DENSE_SKINNY) {
    // Its 16 waves split K inside the block (idle waves when K/128 < 16).
    DWM_UNSUPPORTED_IF(M > 16, "dense_fp8 plan: the skinny kernel takes M <= 16 (M=%lld)", (long long)M);
    DWM_UNSUPPORTED_IF(p.tile_m != 16 || p.tile_n != 16 || p.ksplit != 16 || p.stages != 2,
                       "dense_fp8 plan: the skinny kernel runs 16 x 16 tiles, 16 K runs, ring depth 2");
    return DWM_OK;
  }
  DWM_UNSUPPORTED_IF(p.ksplit < 1 || p.ksplit > KB || p.ksplit > 65535,
                     "dense_fp8 plan: ksplit %d outside [1, K/128 = %lld]", p.ksplit, (long long)KB);
  DWM_UNSUPPORTED_IF(whole_runs(KB, p.ksplit) != p.ksplit, "dense_fp8 plan: ksplit %d leaves an empty K run (K/128 = %lld)",
                     p.ksplit, (long long)KB);
  switch (p.kernel) {
    case DWM_DENSE_MFMA: {
      DWM_UNSUPPORTED_IF(p.tile_n != 128 || (p.tile_m != 128 && p.tile_m != 256),
                         "dense_fp8 plan: MFMA tiles are 128 x 128 or 256 x 128 (got %d x %d)", p.tile_m, p.tile_n);
      DWM_UNSUPPORTED_IF(!dense_mfma_ok(M, K, N, p.tile_m),
                         "dense_fp8 plan: the MFMA kernel needs M > 16, N %% 128 == 0 and 32-bit operand offsets");
      // Ring depths that fit 160 KB of LDS (W8A8's prefetching loop needs 3).
      const bool ok = a8 ? (p.tile_m == 128 ? (p.stages == 3 || p.stages == 4) : p.stages == 3)
                         : (p.tile_m == 128 ? (p.stages >= 2 && p.stages <= 4) : (p.stages == 2 || p.stages == 3));
      DWM_UNSUPPORTED_IF(!ok, "dense_fp8 plan: %s %d-row MFMA tiles have no %d-stage ring", v, p.tile_m, p.stages);
      return DWM_OK;
    }
    case DWM_DENSE_TILED: {
      const bool ok = (p.tile_m == 16 && p.tile_n == 64) || (p.tile_m == 64 && p.tile_n == 128) ||
                      (p.tile_m == 128 && p.tile_n == 128);
      DWM_UNSUPPORTED_IF(!ok || p.stages != 2,
                         "dense_fp8 plan: tiled kernel tiles are 16 x 64, 64 x 128 or 128 x 128 with 2 stages");
      DWM_UNSUPPORTED_IF((M + p.tile_m - 1) / p.tile_m > 65535, "dense_fp8 plan: M too large for %d-row tiles", p.tile_m);
      return DWM_OK;
    }
    default:
      DWM_UNSUPPORTED_IF(true, "dense_fp8 plan: unknown kernel %d", p.kernel);
  }
}

static int64_t plan_workspace(int64_t M, int64_t N, const dwm_dense_plan &p) {
  return (p.kernel != DWM_DENSE_SKINNY && p.ksplit > 1) ? (int64_t)p.ksplit * M * N * 4 : 0;
}

// The plan the last dense call of this thread launched (for tests and traces).
static thread_local dwm_dense_plan t_last_plan{0, 0, 0, 0, 0};

template <class C, bool A8, int NS>
static void launch_mfma(const void *x, const float *sx, int64_t M, int64_t K, int64_t N, const uint8_t *w,
                        const float *sw, int sw_ld, int ks, uint16_t *out, float *partial, hipStream_t st) {
  const dim3 grid((unsigned)(N / C::BN), (unsigned)((M + C::BM - 1) / C::BM), (unsigned)ks);
  hipLaunchKernelGGL((dense_fp8_mfma_kernel<C, A8, NS, A8>), grid, dim3(C::THREADS), 0, st, x, sx, M, (int)K, (int)N,
                     w, sw, sw_ld, ks, out, partial);
}

template <int MB, int NBW, bool A8, bool PRE = false>
static void launch_tiled(const void *x, const float *sx, int64_t M, int64_t K, int64_t N, const uint8_t *w,
                         const float *sw, int sw_ld, int ksplit, uint16_t *out, float *partial, hipStream_t st) {
  const int64_t NT = 64 * NBW, MT = 16 * MB;
  dim3 grid((unsigned)((N + NT - 1) / NT), (unsigned)((M + MT - 1) / MT), (unsigned)ksplit);
  hipLaunchKernelGGL((dense_fp8_kernel<MB, NBW, A8, PRE>), grid, dim3(kDenseThreads), 0, st, x, sx, M, (int)K,
                     (int)N, w, sw, sw_ld, ksplit, out, partial);
}

// The f32 partials [ks][M][N] summed in run order and rounded once.  A grid
// of fewer than 1024 blocks (under four waves per SIMD) issues the loads of
// up to 8 runs per thread before adding them: with N = 4096 and 8 runs, M =
// 48 took 0.7-1.0 us less and M = 128 0.2-0.35 us less.  Larger grids hide
// the latency with their waves (8 runs at a time measured 0.5 us slower at
// M = 256), so they add one run at a time.
template <int KC>
static void launch_reduce_kc(const float *partial, int ks, int64_t MN, uint16_t *out, int64_t blocks, bool vec4,
                             hipStream_t st) {
  if (vec4) hipLaunchKernelGGL(dense_fp8_reduce4_kernel<KC>, dim3((unsigned)blocks), dim3(256), 0, st, partial, ks, MN, out);
  else hipLaunchKernelGGL(dense_fp8_reduce_kernel<KC>, dim3((unsigned)blocks), dim3(256), 0, st, partial, ks, MN, out);
}

static int launch_reduce(const float *partial, int ks, int64_t MN, uint16_t *out, hipStream_t st) {
  const bool vec4 = (((uintptr_t)partial | (uintptr_t)out) & 15) == 0;
  const int64_t threads = vec4 ? MN / 4 : MN;
  const int64_t blocks = (threads + 255) / 256 < 4096 ? (threads + 255) / 256 : 4096;
  if (blocks >= 1024 || ks <= 1) launch_reduce_kc<1>(partial, ks, MN, out, blocks, vec4, st);
  else if (ks <= 2) launch_reduce_kc<2>(partial, ks, MN, out, blocks, vec4, st);
  else if (ks <= 4) launch_reduce_kc<4>(partial, ks, MN, out, blocks, vec4, st);
  else launch_reduce_kc<8>(partial, ks, MN, out, blocks, vec4, st);
  return launch_status("dense_fp8 reduce");
}

// The "pre" rounding runs on the tiled kernel with its own plan for the shape.
static dwm_dense_plan pre_plan(int64_t M, int64_t K, int64_t N) {
  dwm_dense_plan p = tiled_default(M, K, N);
  p.ksplit = whole_runs(K / 128, p.ksplit);
  return p;
}

// Runs one dense GEMM with `plan` (NULL: the default plan).
template <bool A8>
static int run_dense(const void *x, const float *sx, int64_t M, int64_t K, int64_t N, const uint8_t *w,
                     const float *sw, int sw_ld, uint16_t *out, const dwm_dense_plan *plan, void *workspace,
                     int64_t workspace_bytes, hipStream_t st) {
  const dwm_dense_plan p = plan ? *plan : default_plan(M, K, N, A8);
  int rc = check_plan(M, K, N, A8, p);
  if (rc != DWM_OK) return rc;
  const int64_t need = plan_workspace(M, N, p);
  DWM_CHECK_ARG(need == 0 || (workspace && workspace_bytes >= need), "dense_fp8: workspace of %lld bytes needed",
                (long long)need);
  float *const partial = need ? (float *)workspace : nullptr;
  const int ks = p.ksplit;
  if (p.kernel == DWM_DENSE_SKINNY) {
    hipLaunchKernelGGL((dense_fp8_skinny_kernel<16, 2, A8>), dim3((unsigned)(N / 16)), dim3(1024), 0, st, x, sx,
                       (int)M, (int)K, (int)N, w, sw, sw_ld, out);
  } else if (p.kernel == DWM_DENSE_MFMA) {
    if constexpr (A8) {
      if (p.tile_m == 256) launch_mfma<DenseMfmaCfg<4, 2, true>, true, 3>(x, sx, M, K, N, w, sw, sw_ld, ks, out, partial, st);
      else if (p.stages == 3) launch_mfma<DenseMfmaCfg<2, 2, true>, true, 3>(x, sx, M, K, N, w, sw, sw_ld, ks, out, partial, st);
      else launch_mfma<DenseMfmaCfg<2, 2, true>, true, 4>(x, sx, M, K, N, w, sw, sw_ld, ks, out, partial, st);
    } else {
      if (p.tile_m == 256 && p.stages == 2) launch_mfma<DenseMfmaCfg<4, 2, false>, false, 2>(x, sx, M, K, N, w, sw, sw_ld, ks, out, partial, st);
      else if (p.tile_m == 256) launch_mfma<DenseMfmaCfg<4, 2, false>, false, 3>(x, sx, M, K, N, w, sw, sw_ld, ks, out, partial, st);
      else if (p.stages == 2) launch_mfma<DenseMfmaCfg<2, 4, false, 1>, false, 2>(x, sx, M, K, N, w, sw, sw_ld, ks, out, partial, st);
      else if (p.stages == 3) launch_mfma<DenseMfmaCfg<2, 4, false, 1>, false, 3>(x, sx, M, K, N, w, sw, sw_ld, ks, out, partial, st);
      else launch_mfma<DenseMfmaCfg<2, 4, false, 1>, false, 4>(x, sx, M, K, N, w, sw, sw_ld, ks, out, partial, st);
    }
  } else {
    if (p.tile_m == 16) launch_tiled<1, 1, A8>(x, sx, M, K, N, w, sw, sw_ld, ks, out, partial, st);
    else if (p.tile_m == 64) launch_tiled<4, 2, A8>(x, sx, M, K, N, w, sw, sw_ld, ks, out, partial, st);
    else launch_tiled<8, 2, A8>(x, sx, M, K, N, w, sw, sw_ld, ks, out, partial, st);
  }
  rc = launch_status("dense_fp8");
  if (rc != DWM_OK) return rc;
  t_last_plan = p;
  if (!partial) return DWM_OK;
  return launch_reduce(partial, ks, M * N, out, st);
}

static int check_dense(int64_t M, int64_t K, int64_t N) {
  DWM_CHECK_ARG(M >= 0 && K > 0 && N > 0, "dense_fp8: bad sizes M=%lld K=%lld N=%lld", (long long)M, (long long)K,
                (long long)N);
  DWM_UNSUPPORTED_IF(K % 128 != 0 || N % 16 != 0, "dense_fp8: K %% 128 == 0 and N %% 16 == 0 required");
  DWM_UNSUPPORTED_IF(K > (1 << 30) || N > (1 << 30), "dense_fp8: K, N must be < 2^30");
  return DWM_OK;
}

}  // namespace dwm

using namespace dwm;

extern "C" int dwm_dense_fp8_prepack(const uint8_t *w, int64_t K, int64_t N, uint8_t *out, void *stream) {
  clear_error();
  int rc = check_dense(1, K, N);
  if (rc != DWM_OK) return rc;
  DWM_CHECK_ARG(w && out, "dense_fp8_prepack: null pointer");
  DWM_CHECK_ARG((uintptr_t)out % 16 == 0, "dense_fp8_prepack: output must be 16-byte aligned");
  const int64_t total = (N / 16) * (K / 128) * 64;
  hipLaunchKernelGGL(dense_fp8_prepack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), w, K, N, out);
  return launch_status("dense_fp8_prepack");
}

extern "C" int dwm_dense_fp8_plan(int64_t M, int64_t K, int64_t N, int w8a8, dwm_dense_plan *plan) {
  clear_error();
  int rc = check_dense(M, K, N);
  if (rc != DWM_OK) return rc;
  DWM_CHECK_ARG(plan, "dense_fp8_plan: null pointer");
  DWM_UNSUPPORTED_IF(w8a8 && N % 128 != 0, "dense_fp8_w8a8: N %% 128 == 0 required (128x128 weight blocks)");
  *plan = default_plan(M < 1 ? 1 : M, K, N, w8a8 != 0);
  return DWM_OK;
}

extern "C" int dwm_dense_fp8_plan_check(int64_t M, int64_t K, int64_t N, int w8a8, const dwm_dense_plan *plan) {
  clear_error();
  int rc = check_dense(M, K, N);
  if (rc != DWM_OK) return rc;
  DWM_CHECK_ARG(plan, "dense_fp8_plan_check: null pointer");
  DWM_UNSUPPORTED_IF(w8a8 && N % 128 != 0, "dense_fp8_w8a8: N %% 128 == 0 required (128x128 weight blocks)");
  return check_plan(M < 1 ? 1 : M, K, N, w8a8 != 0, *plan);
}

extern "C" int dwm_dense_fp8_plan_workspace_size(int64_t M, int64_t K, int64_t N, const dwm_dense_plan *plan,
                                                 int64_t *bytes) {
  clear_error();
  int rc = check_dense(M, K, N);
  if (rc != DWM_OK) return rc;
  DWM_CHECK_ARG(plan && bytes, "dense_fp8_plan_workspace_size: null pointer");
  *bytes = plan_workspace(M, N, *plan);
  return DWM_OK;
}

extern "C" int dwm_dense_fp8_last_plan(dwm_dense_plan *plan) {
  clear_error();
  DWM_CHECK_ARG(plan, "dense_fp8_last_plan: null pointer");
  *plan = t_last_plan;
  return DWM_OK;
}

extern "C" int dwm_dense_fp8_workspace_size(int64_t M, int64_t K, int64_t N, int64_t *bytes) {
  clear_error();
  int rc = check_dense(M, K, N);
  if (rc != DWM_OK) return rc;
  DWM_CHECK_ARG(bytes, "dense_fp8_workspace_size: null pointer");
  const int64_t m = M < 1 ? 1 : M;
  // the larger of the W8A16 and W8A8 default plans' needs
  int64_t b = plan_workspace(M, N, default_plan(m, K, N, false));
  if (N % 128 == 0) b = max(b, plan_workspace(M, N, default_plan(m, K, N, true)));
  b = max(b, plan_workspace(M, N, pre_plan(m, K, N)));
  *bytes = b;
  return DWM_OK;
}

extern "C" int dwm_dense_fp8_w8a16_plan(const uint16_t *x, int64_t M, int64_t K, int64_t N, const uint8_t *w,
                                        const float *s, uint16_t *out, const dwm_dense_plan *plan, void *workspace,
                                        int64_t workspace_bytes, void *stream) {
  clear_error();
  int rc = check_dense(M, K, N);
  if (rc != DWM_OK) return rc;
  if (M == 0) return DWM_OK;
  DWM_CHECK_ARG(x && w && s && out, "dense_fp8_w8a16: null pointer");
  DWM_CHECK_ARG((uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0, "dense_fp8_w8a16: x and w must be 16-byte aligned");
  return run_dense<false>(x, nullptr, M, K, N, w, s, (int)N, out, plan, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int dwm_dense_fp8_w8a16(const uint16_t *x, int64_t M, int64_t K, int64_t N, const uint8_t *w,
                                   const float *s, uint16_t *out, void *workspace, int64_t workspace_bytes,
                                   void *stream) {
  return dwm_dense_fp8_w8a16_plan(x, M, K, N, w, s, out, nullptr, workspace, workspace_bytes, stream);
}

extern "C" int dwm_dense_fp8_w8a8_plan(const uint8_t *xq, const float *sx, int64_t M, int64_t K, int64_t N,
                                       const uint8_t *w, const float *sw, uint16_t *out, const dwm_dense_plan *plan,
                                       void *workspace, int64_t workspace_bytes, void *stream) {
  clear_error();
  int rc = check_dense(M, K, N);
  if (rc != DWM_OK) return rc;
  if (M == 0) return DWM_OK;
  DWM_UNSUPPORTED_IF(N % 128 != 0, "dense_fp8_w8a8: N %% 128 == 0 required (128x128 weight blocks)");
  DWM_CHECK_ARG(xq && sx && w && sw && out, "dense_fp8_w8a8: null pointer");
  DWM_CHECK_ARG((uintptr_t)xq % 16 == 0 && (uintptr_t)w % 16 == 0, "dense_fp8_w8a8: xq and w must be 16-byte aligned");
  return run_dense<true>(xq, sx, M, K, N, w, sw, (int)(N / 128), out, plan, workspace, workspace_bytes,
                         as_stream(stream));
}

extern "C" int dwm_dense_fp8_w8a8(const uint8_t *xq, const float *sx, int64_t M, int64_t K, int64_t N,
                                  const uint8_t *w, const float *sw, uint16_t *out, void *workspace,
                                  int64_t workspace_bytes, void *stream) {
  return dwm_dense_fp8_w8a8_plan(xq, sx, M, K, N, w, sw, out, nullptr, workspace, workspace_bytes, stream);
}

extern "C" int dwm_dense_fp8_w8a16_pre(const uint16_t *x, int64_t M, int64_t K, int64_t N, const uint8_t *w,
                                       const float *s, uint16_t *out, void *workspace, int64_t workspace_bytes,
                                       void *stream) {
  clear_error();
  int rc = check_dense(M, K, N);
  if (rc != DWM_OK) return rc;
  if (M == 0) return DWM_OK;
  DWM_CHECK_ARG(x && w && s && out, "dense_fp8_w8a16_pre: null pointer");
  DWM_CHECK_ARG((uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0,
                "dense_fp8_w8a16_pre: x and w must be 16-byte aligned");
  const dwm_dense_plan p = pre_plan(M, K, N);
  DWM_UNSUPPORTED_IF((M + p.tile_m - 1) / p.tile_m > 65535, "dense_fp8_w8a16_pre: M too large");
  const int64_t need = plan_workspace(M, N, p);
  DWM_CHECK_ARG(need == 0 || (workspace && workspace_bytes >= need),
                "dense_fp8_w8a16_pre: workspace of %lld bytes needed", (long long)need);
  float *const partial = need ? (float *)workspace : nullptr;
  hipStream_t st = as_stream(stream);
  const int ks = p.ksplit;
  if (p.tile_m == 16) launch_tiled<1, 1, false, true>(x, nullptr, M, K, N, w, s, (int)N, ks, out, partial, st);
  else if (p.tile_m == 64) launch_tiled<4, 2, false, true>(x, nullptr, M, K, N, w, s, (int)N, ks, out, partial, st);
  else launch_tiled<8, 2, false, true>(x, nullptr, M, K, N, w, s, (int)N, ks, out, partial, st);
  rc = launch_status("dense_fp8_w8a16_pre");
  if (rc != DWM_OK) return rc;
  t_last_plan = p;
  if (!partial) return DWM_OK;
  return launch_reduce(partial, ks, M * N, out, st);
}

#ifdef DWTPU_TIMELINE
// Timeline build only: record the MFMA tile kernel's per-wave step accounting
// for waves 0 .. waves - 1 (16 per block) into buf (waves x kDsSlots words,
// zeroed by the caller), or stop (NULL).
extern "C" int dwm_dense_steps_set(uint64_t *buf, int64_t waves) {
  clear_error();
  DWM_CHECK_ARG(waves >= 0 && (buf || waves == 0), "dense_steps_set: bad buffer");
  if (hipMemcpyToSymbol(HIP_SYMBOL(dwm::g_dense_steps), &buf, sizeof(buf)) != hipSuccess ||
      hipMemcpyToSymbol(HIP_SYMBOL(dwm::g_dense_steps_waves), &waves, sizeof(waves)) != hipSuccess)
    return launch_status("dense_steps_set");
  return DWM_OK;
}
#endif
