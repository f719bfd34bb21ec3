// Checkpoint weight formats -> inputs of the hot path (load time).
//
// * MXFP4 expert weights (OCP MX: e2m1 codes two per byte along K, one ue8m0
//   scale per 32 K-values; layout [E, N, K/2] + [E, N, K/32]) -> the fp4
//   gmm's e2m1 codes [E, K, N/2] (two per byte along N) and e8m0 scale codes
//   [E, K/32, N]: the reference dequantizes the checkpoint and requantizes it
//   at block 32 with power-of-two scales (quantize_tensor with
//   power_of_two_scale, patches/tpu-inference/0001-dsv4-v6e-enablement.patch:
//   338-349, called for block-32 e2m1 at 0001-...:558-562), then stores the
//   scales as e8m0 codes when lossless (e8m0_encode,
//   kernels/tpu_inference/layers/common/quantization/e8m0_scale.py:28-35).
// * FP8 weights with 128 x 128 block scales -> e4m3 [K, N] with power-of-two
//   f32 scales per (128-deep K-block, column), the dense fp8 kernel's layout
//   (0001-...:499-512).
//
// Both are one pass over HBM: a block owns a 128 (K) x 64 (N) tile, computes
// each (column, K-block) group's requantization in registers (every f32 step
// in the order the reference takes it: x = code * scale, scale' =
// pow2ceil(absmax / max), code' = rne(x * (1 / scale'))), and transposes the
// tile through LDS so both the reads and the writes are whole 16-byte runs.
#include "common.h"

typedef __attribute__((ext_vector_type(2))) float f32x2_t;

namespace dwm {

// e2m1 nibble -> f32 (sign bit 3; magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6).
__device__ __forceinline__ float e2m1_f32(uint32_t c) {
  const uint32_t e = (c >> 1) & 3u, m = c & 1u;
  const uint32_t mag = e == 0 ? (m ? 0x3F000000u : 0u) : (((e + 126u) << 23) | (m << 22));
  return __builtin_bit_cast(float, mag | ((c & 8u) << 28));
}

// f32 -> e2m1 nibble, round to nearest even, saturating at 6; the sign of q
// (also of -0 and of values rounding to 0) sets bit 3.
__device__ __forceinline__ uint32_t rne_e2m1(float q) {
  const float a = fabsf(q);
  const uint32_t c = (a > 0.25f) + (a >= 0.75f) + (a > 1.25f) + (a >= 1.75f) + (a > 2.5f) + (a >= 3.5f) + (a > 5.0f);
  return c | ((__builtin_bit_cast(uint32_t, q) >> 28) & 8u);
}

// 2^ceil(log2(s)) for finite s > 0, exactly as frexp gives it (mantissa in
// [0.5, 1): a power of two maps to itself); s <= 0 is returned unchanged.
__device__ __forceinline__ float pow2_ceil_f32(float s) {
  if (!(s > 0.0f)) return s;
  const uint32_t b = __builtin_bit_cast(uint32_t, s);
  int32_t e;  // s in (2^(e-1), 2^e]
  const uint32_t ef = b >> 23, m = b & 0x7FFFFFu;
  if (ef != 0) {
    e = (int32_t)ef - 127 + (m != 0 ? 1 : 0);
  } else {  // subnormal: m * 2^-149
    const int32_t p = 31 - __builtin_clz(m);
    e = p - 149 + ((m & (m - 1)) != 0 ? 1 : 0);
  }
  if (e > 127) return __builtin_bit_cast(float, 0x7F800000u);
  if (e >= -126) return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23);
  return __builtin_bit_cast(float, 1u << (e + 149));
}

// 1 / s for a power of two s (exact, or infinite); zero and an infinite
// reciprocal give 0 (a zero block stays zero).
__device__ __forceinline__ float inv_or_zero(float s) {
  if (s == 0.0f) return 0.0f;
  const float inv = 1.0f / s;
  return __builtin_isinf(inv) ? 0.0f : inv;
}

// One MXFP4 group (32 codes of one column, checkpoint scale code sc) ->
// 32 requantized codes (nibble i of word i / 8), the e8m0 scale code, and
// the lossy / finite flags.  For 4 <= sc <= 252 every f32 step is exact and
// the result has a closed form: with v the group's largest e2m1 magnitude,
// the codes move up k = 3, 2, 2, 1, 1, 0, 0 binades (v = .5, 1, 1.5, 2, 3,
// 4, 6) and the scale code down by k; other codes take the f32 path.
struct Mx4Group {
  uint32_t q[4];
  uint32_t scode;
  bool lossy, finite;
};

__device__ __forceinline__ Mx4Group mxfp4_group(u32x4_t in, uint32_t sc) {
  Mx4Group r;
  if (sc >= 4u && sc <= 252u) {
    uint32_t vmax = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t m = in[w] & 0x77777777u;
#pragma unroll
      for (int b = 0; b < 8; ++b) vmax = max(vmax, (m >> (4 * b)) & 7u);
    }
    // k by the largest magnitude index (0: all zero), and each magnitude
    // index's image after the k-binade shift, as nibble tables.
    const uint32_t k = (0x00112233u >> (4 * vmax)) & 3u;
    const uint32_t lut = k == 0 ? 0x76543210u : k == 1 ? 0x00765420u : k == 2 ? 0x00007640u : 0x00000060u;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t o = 0;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const uint32_t c = (in[w] >> (4 * b)) & 0xFu;
        o |= (((lut >> (4 * (c & 7u))) & 7u) | (c & 8u)) << (4 * b);
      }
      r.q[w] = o;
    }
    r.scode = vmax == 0 ? 0u : sc - k;
    r.lossy = false;
    r.finite = true;
    return r;
  }
  // Checkpoint scale 2^(sc - 127): code 0 is 2^-127 (subnormal), 255 is NaN.
  const float s = sc == 255u ? __builtin_bit_cast(float, 0x7FC00000u)
                             : __builtin_bit_cast(float, sc == 0u ? 0x00400000u : sc << 23);
  float x[32];
  float amax = 0.0f;
  bool finite = true;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    x[i] = e2m1_f32((in[i >> 3] >> (4 * (i & 7))) & 0xFu) * s;
    finite = finite && __builtin_isfinite(x[i]);
    amax = fmaxf(amax, fabsf(x[i]));
  }
  const float scale = pow2_ceil_f32(finite ? amax / 6.0f : 0.0f);
  const float inv = inv_or_zero(scale);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t o = 0;
#pragma unroll
    for (int b = 0; b < 8; ++b) o |= (finite ? rne_e2m1(x[8 * w + b] * inv) : 0u) << (4 * b);
    r.q[w] = o;
  }
  const uint32_t sb = __builtin_bit_cast(uint32_t, scale);
  r.scode = finite ? (sb >> 23) & 0xFFu : 255u;
  r.lossy = finite && (((sb & 0x807FFFFFu) != 0) || ((sb >> 23) & 0xFFu) == 255u);
  r.finite = finite;
  return r;
}

__global__ void format_status_zero_kernel(int32_t *status) {
  if (threadIdx.x < 2) status[threadIdx.x] = 0;
}

// Wave-aggregated count of lanes with `flag` into *counter.
__device__ __forceinline__ void count_flags(bool flag, int32_t *counter) {
  const uint64_t m = __ballot(flag);
  if ((threadIdx.x & 63) == 0 && m != 0) atomicAdd(counter, (int32_t)__popcll(m));
}

// ---- MXFP4 --------------------------------------------------------------
// Block (kt, nt, e): K rows kt*128 .. +127, columns nt*64 .. +63 (before the
// optional w13 de-interleave).  Thread t: column n = nt*64 + t/4, K-block
// kt*4 + t%4.
__global__ __launch_bounds__(256) void mxfp4_requant_kernel(const uint8_t *__restrict__ blocks,
                                                            const uint8_t *__restrict__ scales, int64_t N, int64_t K,
                                                            int interleave, uint8_t *__restrict__ codes_out,
                                                            uint8_t *__restrict__ scale_out,
                                                            int32_t *__restrict__ status) {
  __shared__ uint8_t s_code[128][64];
  const int t = threadIdx.x, nl = t >> 2, kbl = t & 3;
  const int64_t e = blockIdx.z, kt = blockIdx.x, nt = blockIdx.y;
  const int64_t n = nt * 64 + nl;
  const int64_t kb = kt * 4 + kbl;
  const u32x4_t in = *(const u32x4_t *)(blocks + (e * N + n) * (K / 2) + kb * 16);
  const Mx4Group g = mxfp4_group(in, scales[(e * N + n) * (K / 32) + kb]);
  const int cn = interleave ? ((nl & 1) ? 32 + (nl >> 1) : (nl >> 1)) : nl;
#pragma unroll
  for (int i = 0; i < 32; ++i) s_code[kbl * 32 + i][cn] = (uint8_t)((g.q[i >> 3] >> (4 * (i & 7))) & 0xFu);
  const uint32_t scode = g.scode;
  const bool lossy = g.lossy, finite = g.finite;
  const int64_t nout = interleave ? ((n & 1) ? N / 2 + (n >> 1) : (n >> 1)) : n;
  scale_out[(e * (K / 32) + kb) * N + nout] = (uint8_t)scode;
  count_flags(lossy, status);
  count_flags(!finite, status + 1);
  __syncthreads();
  // Row kl of the tile, 32 codes of half h -> 16 bytes.
  const int kl = t >> 1, h = t & 1;
  u32x4_t o;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 8; ++b) v |= (uint32_t)s_code[kl][h * 32 + w * 8 + b] << (4 * b);
    o[w] = v;
  }
  const int64_t col = interleave ? (h ? N / 2 : 0) + nt * 32 : nt * 64 + h * 32;
  *(u32x4_t *)(codes_out + (e * K + kt * 128 + kl) * (N / 2) + col / 2) = o;
}

// ---- FP8 128 x 128 -> 1 x 128 ---------------------------------------------
// Block (kb, nt): K rows kb*128 .. +127, columns nt*64 .. +63.  The tile is
// staged [k][n] in LDS; thread t then owns column t/4, rows 32*(t%4) .. +31.
// Four e4m3 codes (one dword) -> f32, exactly (the gfx950 converter with
// unit scale decodes OCP e4m3 exactly, NaN codes included).
__device__ __forceinline__ void e4m3x4_f32(uint32_t w, float *v) {
  const f32x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, false);
  const f32x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, true);
  v[0] = lo[0];
  v[1] = lo[1];
  v[2] = hi[0];
  v[3] = hi[1];
}

// FP8 block requant, block (kb, nt): K rows kb*128 .. +127, columns nt*64 ..
// +63.  Thread t: column nl = t / 4, K part t % 4 (32 values).  With the
// checkpoint's [N, K] layout the thread loads exactly its own 32 codes; the
// [K, N] layout is transposed through LDS first.  The new codes leave
// through the LDS tile as whole 32-byte runs of output rows.
__global__ __launch_bounds__(256) void fp8_block_requant_kernel(const uint8_t *__restrict__ w,
                                                                const float *__restrict__ scale, int64_t K, int64_t N,
                                                                int input_nk, uint8_t *__restrict__ w_out,
                                                                float *__restrict__ scale_out,
                                                                int32_t *__restrict__ status) {
  __shared__ __attribute__((aligned(16))) uint8_t s_t[128][64];
  const int t = threadIdx.x;
  const int64_t kb = blockIdx.x, nt = blockIdx.y;
  const int nl = t >> 2, part = t & 3;
  uint32_t cw[8];  // the thread's 32 input codes, k = part * 32 + 4 j .. + 3 in word j
  if (input_nk) {
    const uint8_t *src = w + (nt * 64 + nl) * K + kb * 128 + part * 32;
    const u32x4_t a = *(const u32x4_t *)src, b = *(const u32x4_t *)(src + 16);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      cw[j] = a[j];
      cw[4 + j] = b[j];
    }
  } else {
    const int kl = t >> 1, h = t & 1;
    const uint8_t *src = w + (kb * 128 + kl) * N + nt * 64 + h * 32;
    *(u32x4_t *)&s_t[kl][h * 32] = *(const u32x4_t *)src;
    *(u32x4_t *)&s_t[kl][h * 32 + 16] = *(const u32x4_t *)(src + 16);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t v = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) v |= (uint32_t)s_t[part * 32 + 4 * j + q][nl] << (8 * q);
      cw[j] = v;
    }
  }
  const int64_t n = nt * 64 + nl;
  const float bs = input_nk ? scale[(n / 128) * (K / 128) + kb] : scale[kb * (N / 128) + n / 128];
  float x[32];
  float amax = 0.0f;
  bool finite = true;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    e4m3x4_f32(cw[j], x + 4 * j);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      x[4 * j + q] *= bs;
      finite = finite && __builtin_isfinite(x[4 * j + q]);
      amax = fmaxf(amax, fabsf(x[4 * j + q]));
    }
  }
  // The four threads of a column are adjacent lanes.
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  int fin = finite ? 1 : 0;
  fin &= __shfl_xor(fin, 1, 64);
  fin &= __shfl_xor(fin, 2, 64);
  const bool all_finite = fin != 0;
  const float s2 = pow2_ceil_f32(all_finite ? amax / 448.0f : 0.0f);
  const float inv = inv_or_zero(s2);
  bool exact = true;
  uint32_t qw[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float y[4], back[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) y[q] = x[4 * j + q] * inv;
    qw[j] = all_finite ? f32x4_e4m3(y) : 0u;
    e4m3x4_f32(qw[j], back);
#pragma unroll
    for (int q = 0; q < 4; ++q) exact = exact && (back[q] * s2 == x[4 * j + q]);
  }
  int ex = exact ? 1 : 0;
  ex &= __shfl_xor(ex, 1, 64);
  ex &= __shfl_xor(ex, 2, 64);
  __syncthreads();  // every thread has read its inputs before codes overwrite the tile
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) s_t[part * 32 + 4 * j + q][nl] = (uint8_t)(qw[j] >> (8 * q));
  if (part == 0) scale_out[kb * N + n] = all_finite ? s2 : __builtin_bit_cast(float, 0x7FC00000u);
  count_flags(part == 0 && all_finite && !ex, status);
  count_flags(part == 0 && !all_finite, status + 1);
  __syncthreads();
  const int kl = t >> 1, h = t & 1;
  uint8_t *dst = w_out + (kb * 128 + kl) * N + nt * 64 + h * 32;
  *(u32x4_t *)dst = *(const u32x4_t *)&s_t[kl][h * 32];
  *(u32x4_t *)(dst + 16) = *(const u32x4_t *)&s_t[kl][h * 32 + 16];
}

// ---- Tiled MXFP4 (K % 256 == 0, N % 256 == 0): whole 128-byte input rows
// per 8 lanes and whole 128-byte output rows per 8 lanes, the transpose
// staged in LDS.

// Wave-aggregated add of a per-lane count into *counter.
__device__ __forceinline__ void count_add(int v, int32_t *counter) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  if ((threadIdx.x & 63) == 0 && v != 0) atomicAdd(counter, v);
}

// MXFP4, block (kt, nt, e): K rows kt*256 .. +255, columns nt*256 .. +255.
// Thread t: column octet o = t / 8 (columns 8 o .. 8 o + 7), K-block t % 8.
// Its 32 x 8 codes are packed per row into words of 8 nibbles and staged as
// s_out[kb][i][o] (kb blocks padded by 8 words: conflict-free writes).
// In-register transpose of an 8 x 8 matrix of nibbles, element (r, s) =
// nibble s of x[r] -> nibble r of x[s]: three rounds of block swaps (2 x 2,
// 4 x 4, 8 x 8 blocks), the bit-matrix transpose of Hacker's Delight
// (section 7-3) on 4-bit elements.
__device__ __forceinline__ void transpose8x8_nibbles(uint32_t *x) {
#pragma unroll
  for (int r = 0; r < 8; r += 2) {
    const uint32_t t = ((x[r] >> 4) ^ x[r + 1]) & 0x0F0F0F0Fu;
    x[r + 1] ^= t;
    x[r] ^= t << 4;
  }
#pragma unroll
  for (int r = 0; r < 8; r += (r & 1) ? 3 : 1) {  // r = 0, 1, 4, 5
    const uint32_t t = ((x[r] >> 8) ^ x[r + 2]) & 0x00FF00FFu;
    x[r + 2] ^= t;
    x[r] ^= t << 8;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t t = ((x[r] >> 16) ^ x[r + 4]) & 0x0000FFFFu;
    x[r + 4] ^= t;
    x[r] ^= t << 16;
  }
}

__global__ __launch_bounds__(256) void mxfp4_requant_tile_kernel(const uint8_t *__restrict__ blocks,
                                                                 const uint8_t *__restrict__ scales, int64_t N,
                                                                 int64_t K, int interleave,
                                                                 uint8_t *__restrict__ codes_out,
                                                                 uint8_t *__restrict__ scale_out,
                                                                 int32_t *__restrict__ status) {
  constexpr int KBW = 32 * 32 + 8;  // words per K-block of s_out
  __shared__ __attribute__((aligned(16))) uint32_t s_out[8 * KBW];
  __shared__ __attribute__((aligned(16))) uint8_t s_sc[8][256];
  const int t = threadIdx.x, o = t >> 3, kb = t & 7;
  const int64_t e = blockIdx.z, k0 = (int64_t)blockIdx.x * 256, n0 = (int64_t)blockIdx.y * 256;
  uint32_t qc[4][8];  // qc[j][c]: codes k = 8 j .. 8 j + 7 (nibbles) of column c
  uint32_t sc_lo = 0, sc_hi = 0;
  int nlossy = 0, nnonfinite = 0;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int64_t n = n0 + 8 * o + c;
    const u32x4_t in = *(const u32x4_t *)(blocks + (e * N + n) * (K / 2) + k0 / 2 + kb * 16);
    const Mx4Group g = mxfp4_group(in, scales[(e * N + n) * (K / 32) + k0 / 32 + kb]);
#pragma unroll
    for (int j = 0; j < 4; ++j) qc[j][c] = g.q[j];
    const uint32_t scode = g.scode;
    nlossy += g.lossy ? 1 : 0;
    nnonfinite += g.finite ? 0 : 1;
    if (c < 4) sc_lo |= scode << (8 * c);
    else sc_hi |= scode << (8 * (c - 4));
  }
  // ow[i]: the 8 columns' codes of row k = i, column c in nibble c; with
  // interleave the columns are taken in the order 0, 2, 4, 6, 1, 3, 5, 7, so
  // the low half-word holds the even (w1) and the high one the odd (w3) codes.
  uint32_t ow[32];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t x[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) x[c] = interleave ? qc[j][(c < 4) ? 2 * c : 2 * (c - 4) + 1] : qc[j][c];
    transpose8x8_nibbles(x);
#pragma unroll
    for (int r = 0; r < 8; ++r) ow[8 * j + r] = x[r];
  }
  if (!interleave) {
#pragma unroll
    for (int i = 0; i < 32; ++i) s_out[kb * KBW + i * 32 + o] = ow[i];
    *(uint32_t *)&s_sc[kb][8 * o] = sc_lo;
    *(uint32_t *)&s_sc[kb][8 * o + 4] = sc_hi;
  } else {
    // Even columns (w1) go to the first half of the output, odd (w3) to the
    // second: this octet's even / odd codes are positions 4 o .. 4 o + 3.
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      uint16_t *row = (uint16_t *)&s_out[kb * KBW + i * 32];
      row[o] = (uint16_t)(ow[i] & 0xFFFFu);
      row[32 + o] = (uint16_t)(ow[i] >> 16);
    }
    const uint32_t sev = (sc_lo & 0xFFu) | ((sc_lo >> 8) & 0xFF00u) | ((sc_hi << 16) & 0xFF0000u) | ((sc_hi << 8) & 0xFF000000u);
    const uint32_t sod = ((sc_lo >> 8) & 0xFFu) | ((sc_lo >> 16) & 0xFF00u) | ((sc_hi << 8) & 0xFF0000u) | (sc_hi & 0xFF000000u);
    *(uint32_t *)&s_sc[kb][4 * o] = sev;
    *(uint32_t *)&s_sc[kb][128 + 4 * o] = sod;
  }
  count_add(nlossy, status);
  count_add(nnonfinite, status + 1);
  __syncthreads();
  // 256 output rows of 128 bytes, 8 lanes per row.
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int row = 32 * p + (t >> 3), ch = t & 7;
    const u32x4_t v = *(const u32x4_t *)&s_out[(row >> 5) * KBW + (row & 31) * 32 + ch * 4];
    const int64_t colbyte = interleave ? (ch < 4 ? 0 : N / 4) + (n0 / 2) / 2 + (ch & 3) * 16 : n0 / 2 + ch * 16;
    __builtin_nontemporal_store(v, (u32x4_t *)(codes_out + (e * K + k0 + row) * (N / 2) + colbyte));
  }
  // 8 rows of 256 scale codes, 16 lanes per row.
  if (t < 128) {
    const int row = t >> 4, ch = t & 15;
    const u32x4_t v = *(const u32x4_t *)&s_sc[row][ch * 16];
    const int64_t col = interleave ? (ch < 8 ? 0 : N / 2) + n0 / 2 + (ch & 7) * 16 : n0 + ch * 16;
    *(u32x4_t *)(scale_out + (e * (K / 32) + k0 / 32 + row) * N + col) = v;
  }
}

}  // namespace dwm

using namespace dwm;

extern "C" int dwm_mxfp4_requant(const uint8_t *blocks, const uint8_t *scales, int64_t E, int64_t N, int64_t K,
                                 int w13_interleave, uint8_t *codes_out, uint8_t *scale_codes_out, int32_t *status,
                                 void *stream) {
  clear_error();
  DWM_CHECK_ARG(E >= 0 && N >= 0 && K >= 0, "mxfp4_requant: bad sizes E=%lld N=%lld K=%lld", (long long)E,
                (long long)N, (long long)K);
  DWM_UNSUPPORTED_IF(K % 128 != 0 || N % 64 != 0, "mxfp4_requant: K %% 128 == 0 and N %% 64 == 0 required");
  DWM_UNSUPPORTED_IF(w13_interleave && N % 128 != 0, "mxfp4_requant: w13_interleave needs N %% 128 == 0");
  DWM_UNSUPPORTED_IF(K / 128 > 0x7FFFFFFF || N / 64 > 65535 || E > 65535, "mxfp4_requant: too large");
  DWM_CHECK_ARG(status != nullptr, "mxfp4_requant: null status");
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(format_status_zero_kernel, dim3(1), dim3(64), 0, st, status);
  if (E == 0 || N == 0 || K == 0) return launch_status("mxfp4_requant");
  DWM_CHECK_ARG(blocks && scales && codes_out && scale_codes_out, "mxfp4_requant: null pointer");
  DWM_CHECK_ARG((uintptr_t)blocks % 16 == 0 && (uintptr_t)codes_out % 16 == 0,
                "mxfp4_requant: blocks and codes_out must be 16-byte aligned");
  if (K % 256 == 0 && N % 256 == 0)
    hipLaunchKernelGGL(mxfp4_requant_tile_kernel, dim3((unsigned)(K / 256), (unsigned)(N / 256), (unsigned)E),
                       dim3(256), 0, st, blocks, scales, N, K, w13_interleave ? 1 : 0, codes_out, scale_codes_out,
                       status);
  else
    hipLaunchKernelGGL(mxfp4_requant_kernel, dim3((unsigned)(K / 128), (unsigned)(N / 64), (unsigned)E), dim3(256),
                       0, st, blocks, scales, N, K, w13_interleave ? 1 : 0, codes_out, scale_codes_out, status);
  return launch_status("mxfp4_requant");
}

extern "C" int dwm_fp8_block_requant(const uint8_t *w, const float *scale, int64_t K, int64_t N, int input_nk,
                                     uint8_t *w_out, float *scale_out, int32_t *status, void *stream) {
  clear_error();
  DWM_CHECK_ARG(K >= 0 && N >= 0, "fp8_block_requant: bad sizes K=%lld N=%lld", (long long)K, (long long)N);
  DWM_UNSUPPORTED_IF(K % 128 != 0 || N % 128 != 0, "fp8_block_requant: K %% 128 == 0 and N %% 128 == 0 required");
  DWM_UNSUPPORTED_IF(K / 128 > 0x7FFFFFFF || N / 64 > 65535, "fp8_block_requant: too large");
  DWM_CHECK_ARG(status != nullptr, "fp8_block_requant: null status");
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(format_status_zero_kernel, dim3(1), dim3(64), 0, st, status);
  if (K == 0 || N == 0) return launch_status("fp8_block_requant");
  DWM_CHECK_ARG(w && scale && w_out && scale_out, "fp8_block_requant: null pointer");
  DWM_CHECK_ARG((uintptr_t)w % 16 == 0 && (uintptr_t)w_out % 16 == 0 && (uintptr_t)scale % 4 == 0,
                "fp8_block_requant: w and w_out must be 16-byte aligned");
  hipLaunchKernelGGL(fp8_block_requant_kernel, dim3((unsigned)(K / 128), (unsigned)(N / 64)), dim3(256), 0, st, w,
                       scale, K, N, input_nk ? 1 : 0, w_out, scale_out, status);
  return launch_status("fp8_block_requant");
}
