// MX mode of the ragged grouped matmul: the lhs quantized to OCP e4m3 with
// one e8m0 scale per 32 values along K, the prepacked e2m1 weights with their
// e8m0 block-32 scales, contracted by the gfx950 scaled MFMA
// v_mfma_scale_f32_32x32x64_f8f6f4 (A = e4m3, B = e2m1, both block scales
// applied in the instruction), f32 accumulation.  This is gmm_v2 with
// lhs_quant_dtype = float8_e4m3fn: the lhs quantization tokamax applies when
// the chip has a native low-precision matrix path
// (patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:89-100), with the
// reference's own power-of-two block quantizer (quantize_tensor,
// patches/tpu-inference/0001-dsv4-v6e-enablement.patch:315-350) at block 32.
//
// mx_quant_e4m3_kernel: bf16 [rows, K] -> e4m3 codes [rows, K] + e8m0 scale
// codes [rows, K/32].  Per 32-value block: exponent e = the smallest with
// absmax <= 448 * 2^e (from absmax's exponent and mantissa bits, no
// rounding), clamped to >= -126; codes = RNE e4m3 of x * 2^-e (the gfx950
// converter at unit scale, exact RNE); scale code e + 127.  A block holding
// a NaN or an infinity gets codes 0x7F and scale code 255.
//
// gmm_mx_kernel (K < 4096) and gmm_mx128_kernel (K >= 4096, 128-deep steps,
// described with its config below): the tile scheduler, warp
// specialisation and epilogue of the bf16 kernel (gmm_fp4.hip,
// gmm_tiles.h), with these data per 64-deep K step of a 96 x 512 tile:
//   A   96 rows x 64 bytes of e4m3 codes (chunk c of row r at physical chunk
//       c ^ ((r >> 2) & 3): the 16 rows one LDS cycle reads hit 16 distinct
//       16-byte bank groups);
//   W   the 8 column groups' prepacked e2m1 codes, 2 KiB each (fp4.hip);
// and, in even steps only (one dword covers a 128-deep block):
//   AS  the lhs scale dword of each row (K-blocks 4 kb .. 4 kb + 3);
//   S   the weight scale dword of each group lane (fp4.hip's scale layout).
// The MFMA's operands need no conversion: lane (c, h) of a weight group's
// 1 KiB half holds the 32 codes of column c at k = 32 h .. 32 h + 31 of the
// step -- the e2m1 B operand of the 32x32x64 MFMA -- and byte 2 f + j of its
// scale dword is that column's scale for K-block h of step 2 kb + f, the
// MFMA's B scale (opsel j).  The e4m3 A operand of lane (r, h) is row r,
// k = 16 h .. + 15 and 32 + 16 h .. + 15; its scale is row r's K-block h.
#include "gmm_tiles.h"

namespace dwm {

typedef __attribute__((ext_vector_type(8))) int i32x8_t;

constexpr int kMxBlock = 32;
constexpr int kMxMinExp = -126;
// K at and above which the 128-deep kernel runs.  Measured on MI355X with
// 96 x 512 tiles: at K = 7168 it is faster than the 64-deep kernel (prefill
// 1.70 -> 1.53 ms, decode gate/up 96 -> 88 us: half the barriers per MFMA),
// at K = 2048 slower (decode down 107 -> 116 us: 16 steps leave too little
// to pipeline behind one step in flight).
constexpr int kMx128MinK = 4096;

// ---------------------------------------------------------------------------
// Quantization.  Thread i handles values 8 i .. 8 i + 7 of the flat [rows, K]
// array; the 4 threads of a 32-value block are consecutive lanes.

// The smallest e >= -126 with a <= 448 * 2^e, for finite a >= 0.
__device__ __forceinline__ int mx_exponent(float a) {
  const uint32_t u = __builtin_bit_cast(uint32_t, a);
  const int ef = (int)(u >> 23);
  if (ef == 0) return kMxMinExp;  // zero or subnormal: far below 448 * 2^-126
  // a = (1 + m / 2^23) 2^(ef - 127) <= 1.75 * 2^(8 + e)
  const int e = ef - 127 - 8 + ((u & 0x7FFFFFu) > 0x600000u ? 1 : 0);
  return e < kMxMinExp ? kMxMinExp : e;
}

__global__ __launch_bounds__(256) void mx_quant_e4m3_kernel(const uint16_t *__restrict__ x, int64_t n8,
                                                            uint8_t *__restrict__ codes,
                                                            uint8_t *__restrict__ scales) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  // n8 is a multiple of 4, so the 4 lanes of a block enter and leave the
  // loop together and the quad shuffles read active lanes.
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
    const u32x4_t raw = __builtin_nontemporal_load((const u32x4_t *)(x + 8 * i));
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = bf16_bits_to_f32(raw[j] & 0xFFFFu);
      v[2 * j + 1] = bf16_bits_to_f32(raw[j] >> 16);
    }
    float amax = 0.0f;
    int bad = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float a = fabsf(v[j]);
      bad |= !(a <= 3.4028234663852886e38f);  // NaN or infinity
      amax = fmaxf(amax, bad ? 0.0f : a);
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    bad |= __shfl_xor(bad, 1, 64);
    bad |= __shfl_xor(bad, 2, 64);
    const int e = mx_exponent(amax);
    uint32_t w0 = 0x7F7F7F7Fu, w1 = 0x7F7F7F7Fu;
    if (!bad) {
      float q[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) q[j] = ldexpf(v[j], -e);  // exact: |q| <= 448
      w0 = f32x4_e4m3(q);
      w1 = f32x4_e4m3(q + 4);
    }
    *(u32x2_t *)(codes + 8 * i) = u32x2_t{w0, w1};
    if ((i & 3) == 0) scales[i >> 2] = (uint8_t)(bad ? 255 : e + 127);
  }
}

// MXFP4 lhs: the smallest e >= -126 with a <= 6 * 2^e, for finite a >= 0
// (a = (1 + m / 2^23) 2^(ef - 127) <= 1.5 * 2^(2 + e)).
__device__ __forceinline__ int mx_exponent_e2m1(float a) {
  const uint32_t u = __builtin_bit_cast(uint32_t, a);
  const int ef = (int)(u >> 23);
  if (ef == 0) return kMxMinExp;  // zero or subnormal: far below 6 * 2^-126
  const int e = ef - 129 + ((u & 0x7FFFFFu) > 0x400000u ? 1 : 0);
  return e < kMxMinExp ? kMxMinExp : e;
}

// |q| <= 6 -> e2m1 nibble, round to nearest even (magnitudes 0, .5, 1, 1.5
// in steps of .5, then 2, 3, 4 in steps of 1, then 4, 6; every difference
// below is exact), sign in bit 3.
__device__ __forceinline__ uint32_t f32_e2m1(float q) {
  const float a = fabsf(q);
  uint32_t c;
  if (a < 2.0f) c = (uint32_t)__builtin_rintf(a * 2.0f);
  else if (a < 4.0f) c = 4u + (uint32_t)__builtin_rintf(a - 2.0f);
  else c = 6u + (uint32_t)__builtin_rintf((a - 4.0f) * 0.5f);
  return c | ((__builtin_bit_cast(uint32_t, q) >> 28) & 8u);
}

// bf16 [rows, K] -> e2m1 codes [rows, K / 2] (value 2 j in the low nibble
// of byte j) + e8m0 scale codes [rows, K / 32]: per 32-value block the
// exponent of mx_exponent_e2m1(absmax), codes = RNE e2m1 of x * 2^-e (exact
// rescale); a block holding a NaN or an infinity gets codes 0 and scale code
// 255.  Thread i handles values 8 i .. 8 i + 7 (4 threads per block).
__global__ __launch_bounds__(256) void mx_quant_e2m1_kernel(const uint16_t *__restrict__ x, int64_t n8,
                                                            uint8_t *__restrict__ codes,
                                                            uint8_t *__restrict__ scales) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
    const u32x4_t raw = __builtin_nontemporal_load((const u32x4_t *)(x + 8 * i));
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = bf16_bits_to_f32(raw[j] & 0xFFFFu);
      v[2 * j + 1] = bf16_bits_to_f32(raw[j] >> 16);
    }
    float amax = 0.0f;
    int bad = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float a = fabsf(v[j]);
      bad |= !(a <= 3.4028234663852886e38f);  // NaN or infinity
      amax = fmaxf(amax, bad ? 0.0f : a);
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    bad |= __shfl_xor(bad, 1, 64);
    bad |= __shfl_xor(bad, 2, 64);
    const int e = mx_exponent_e2m1(amax);
    uint32_t w = 0u;
    if (!bad) {
#pragma unroll
      for (int j = 0; j < 8; ++j) w |= f32_e2m1(ldexpf(v[j], -e)) << (4 * j);  // exact: |x 2^-e| <= 6
    }
    *(uint32_t *)(codes + 4 * i) = w;
    if ((i & 3) == 0) scales[i >> 2] = (uint8_t)(bad ? 255 : e + 127);
  }
}

// ---------------------------------------------------------------------------
// The MX tile kernel.

// RH = 2 stacks two row halves: the tile is (32 MB x 2 rows) x (64 CW / 2
// columns), consumer cw owning column group cw % GT of row half cw / GT (the
// two consumers of a SIMD, cw and cw + 4, then hold both halves).  A group
// of up to 192 rows then reads its weights once, not once per 96 rows.
// AF4: the lhs is e2m1 (MXFP4: 32 bytes per row and 64-deep step, one
// 16-byte A operand per lane, A format 4 in the MFMA) instead of e4m3 (64
// bytes per row and step).
template <int MB, int CW, int NP, int NS, int RH = 1, bool AF4 = false>
struct MxCfg {
  static constexpr int CONS = CW, NPROD = NP, STAGES = NS, HALVES = RH;
  static constexpr bool A_FP4 = AF4;
  static constexpr int GT = CW / RH;                     // 64-column groups per tile
  static constexpr int THREADS = 64 * (CW + NP);
  static constexpr int NT = 64 * GT;
  static constexpr int CMB = MB;                         // 32-row blocks of one consumer
  static constexpr int TMB = MB * RH;                    // 32-row blocks of the tile
  static constexpr int ROWS = 32 * TMB;
  static constexpr int AB = AF4 ? 32 : 64;               // lhs bytes per row and step
  static constexpr int RL = 1024 / AB;                   // rows per 1 KiB lhs load
  static constexpr int W = 0;                            // group i: 2 KiB at W + 2048 i
  static constexpr int A = GT * 2048;                    // ROWS x AB bytes
  static constexpr int AS = A + ROWS * AB;               // 128-row groups x 256 bytes (dword per row)
  static constexpr int AS_LOADS = (ROWS + 63) / 64;      // 256-byte row-scale loads per even step
  static constexpr int S = AS + AS_LOADS * 256;          // group i: 256 bytes at S + 256 i
  static constexpr int STAGE = S + GT * 256;
  static constexpr int A_GROUPS = ROWS / RL;             // 1 KiB lhs loads (RL rows) per step
  static constexpr int G_LOADS = GT / NP;                // weight groups per producer
  static constexpr int AHEAD = 2;                        // steps published per barrier
  static constexpr int EP_STRIDE = 72;
  static_assert(ROWS % RL == 0 && G_LOADS * NP == GT && GT * RH == CW, "load split");
  static_assert(AS_LOADS <= NP, "one row-scale load per producer at most");
  static constexpr int INFLIGHT = NS - 1 - AHEAD;        // steps loading behind the published pair
  static_assert(INFLIGHT >= 1, "stage count");
  static_assert(CW * 32 * EP_STRIDE * 4 <= NS * STAGE, "epilogue staging fits the stages");
};

__device__ __forceinline__ int mx_swizzle(int r) { return (r >> 2) & 3; }
// e2m1 rows hold two 16-byte chunks: rows r and r + 8 of one LDS cycle's 16
// swap them, so the cycle's 16 reads hit 16 distinct 16-byte bank groups.
__device__ __forceinline__ int mx_swizzle4(int r) { return (r >> 3) & 1; }
template <class C>
__device__ __forceinline__ int mx_swz(int r) { return C::A_FP4 ? mx_swizzle4(r) : mx_swizzle(r); }

// Producer wave pw: its lhs row groups are pw, pw + NP, ... (< A_GROUPS); NA
// of them hold rows of the tile (the others are zero in every stage).
// The last AS_LOADS producers (those with fewer lhs row groups) also load
// row-scale dwords, 64 rows each.
template <class C, int NA, bool ASL>
__device__ __forceinline__ void mx_producer(const uint8_t *__restrict__ lhs, const uint8_t *__restrict__ lsc,
                                            const int32_t *__restrict__ row_idx, int64_t lhs_rows, int64_t row0,
                                            int rows, int K, int T, int KB, const uint8_t *__restrict__ wexp,
                                            const uint8_t *__restrict__ sexp, int g0, int G, uint8_t *s_lds,
                                            int pw) {
  constexpr int NP = C::NPROD, NS = C::STAGES;
  constexpr int MAXA = (C::A_GROUPS + NP - 1) / NP;
  constexpr int L_ODD = NA + 2 * C::G_LOADS;
  constexpr int L_EVEN = L_ODD + C::G_LOADS + (ASL ? 1 : 0);
  // Before barrier t the loads of steps t + 2 .. t + NS - 2 may be pending:
  // INFLIGHT steps alternating in parity from t's.
  constexpr int P_HI = (C::INFLIGHT + 1) / 2, P_LO = C::INFLIGHT / 2;
  constexpr int PENDING_T_EVEN = P_HI * L_EVEN + P_LO * L_ODD;
  constexpr int PENDING_T_ODD = P_LO * L_EVEN + P_HI * L_ODD;
  static_assert(PENDING_T_EVEN < 64 && PENDING_T_ODD < 64, "vmcnt range");
  const int lane = threadIdx.x & 63;
  for (int i = NA; i < MAXA; ++i) {
    const int ga = pw + NP * i;
    if (ga < C::A_GROUPS) {
#pragma unroll
      for (int st = 0; st < NS; ++st)
        *(u32x4_t *)(s_lds + st * C::STAGE + C::A + ga * 1024 + lane * 16) = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
  const int KS = K / kMxBlock;  // row-scale bytes per row
  auto src_row = [&](int r) -> int64_t {
    const int rs = r < rows ? r : rows - 1;
    return row_idx ? gather_index(row_idx[row0 + rs], lhs_rows) : row0 + rs;
  };
  // lhs load i: rows RL (pw + NP i) .. + RL - 1; lane l fills physical
  // chunk l % LPR of row + l / LPR with the logical chunk of the swizzle.
  constexpr int LPR = C::AB / 16;                 // 16-byte chunks per row and step
  const int64_t KR = C::A_FP4 ? K / 2 : K;        // lhs bytes per row
  uint32_t aoff[NA > 0 ? NA : 1];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int r = C::RL * (pw + NP * i) + lane / LPR;
    aoff[i] = (uint32_t)(src_row(r) * KR) + (uint32_t)(((lane % LPR) ^ mx_swz<C>(r)) << 4);
  }
  const int aspart = pw - (NP - C::AS_LOADS);  // row-scale load of producers NP - AS_LOADS .. NP - 1
  const uint32_t asoff = ASL ? (uint32_t)(src_row(64 * aspart + lane) * KS) : 0u;
  const uint8_t *wsrc[C::G_LOADS];
  const uint8_t *ssrc[C::G_LOADS];
#pragma unroll
  for (int c = 0; c < C::G_LOADS; ++c) {
    const int g = min(g0 + pw + NP * c, G - 1);  // groups past N feed unstored columns
    wsrc[c] = wexp + (int64_t)g * T * 2048 + lane * 16;
    ssrc[c] = sexp + (int64_t)g * KB * 256 + lane * 4;
  }
  auto issue = [&](int stage, int t) {
    uint8_t *const st = s_lds + stage * C::STAGE;
    const uint8_t *const a = lhs + (int64_t)t * C::AB;
#pragma unroll
    for (int i = 0; i < NA; ++i)
      __builtin_amdgcn_global_load_lds((const void *)(a + aoff[i]),
                                       (lds_void_t *)(st + C::A + (pw + NP * i) * 1024), 16, 0, 0);
#pragma unroll
    for (int c = 0; c < C::G_LOADS; ++c) {
      const int gi = pw + NP * c;
      const uint8_t *const w = wsrc[c] + (int64_t)t * 2048;
      __builtin_amdgcn_global_load_lds((const void *)w, (lds_void_t *)(st + C::W + gi * 2048), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void *)(w + 1024), (lds_void_t *)(st + C::W + gi * 2048 + 1024), 16,
                                       0, 0);
    }
    if ((t & 1) == 0) {
#pragma unroll
      for (int c = 0; c < C::G_LOADS; ++c)
        __builtin_amdgcn_global_load_lds((const void *)(ssrc[c] + (int64_t)(t >> 1) * 256),
                                         (lds_void_t *)(st + C::S + (pw + NP * c) * 256), 4, 0, 0);
      if (ASL)
        __builtin_amdgcn_global_load_lds((const void *)(lsc + asoff + (t >> 1) * 4),
                                         (lds_void_t *)(st + C::AS + aspart * 256), 4, 0, 0);
    }
  };
  // Steps past the last one repeat the last step of the same parity, so
  // every pair of consecutive steps issues the same loads.
  auto clampt = [&](int t) { return t < T ? t : T - 2 + (t & 1); };
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) issue(t, clampt(t));
  int refill = NS - 1;
  for (int t = 0; t < T; ++t) {
    // Steps t, t + 1 have landed once at most the loads of t + 2 .. t + NS - 2
    // are pending.
    if (t & 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(PENDING_T_ODD));
    else __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(PENDING_T_EVEN));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(refill, clampt(t + NS - 1));
    refill = refill == NS - 1 ? 0 : refill + 1;
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
}

// Consumer cw of column group cg, tile rows rb .. rb + rows - 1 (its row half).
template <class C, int AM, bool ACT>
__device__ __forceinline__ void mx_consumer(int T, uint8_t *s_lds, int cw, int cg, int rb, int64_t row0, int rows,
                                            int64_t col0, int N, void *__restrict__ out, int out_f32,
                                            const void *bias, const GmmEpilogue &ep) {
  constexpr int NS = C::STAGES;
  const int lane = threadIdx.x & 63, c32 = lane & 31, h = lane >> 5;
  f32x16_t acc[AM][2];
#pragma unroll
  for (int mb = 0; mb < AM; ++mb)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][j][r] = 0.0f;
  const int woff = C::W + cg * 2048 + lane * 16;
  const int soff = C::S + cg * 256 + lane * 4;
  // A fragment of row block mb: row rb + mb * 32 + c32 (same swizzle for all
  // mb, rb % 16 == 0), logical chunks h and 2 + h (e4m3: k = 16 h .. + 15
  // and 32 + 16 h .. + 15), or chunk h alone (e2m1: k = 32 h .. + 31).
  const int sw = mx_swz<C>(c32);
  const int alo = C::A + (rb + c32) * C::AB + ((h ^ sw) << 4);
  const int ahi = C::A + (rb + c32) * C::AB + (((2 + h) ^ sw) << 4);
  u32x4_t wn[2];
  uint32_t sn = 0, asn[AM];
  i32x8_t an;
  auto read_w = [&](const uint8_t *st) {
    wn[0] = *(const u32x4_t *)(st + woff);
    wn[1] = *(const u32x4_t *)(st + woff + 1024);
  };
  auto read_s = [&](const uint8_t *st) {  // even steps: scale dwords of this and the next step
    sn = *(const uint32_t *)(st + soff);
#pragma unroll
    for (int mb = 0; mb < AM; ++mb) asn[mb] = *(const uint32_t *)(st + C::AS + (rb + mb * 32 + c32) * 4);
  };
  auto read_a = [&](const uint8_t *st, int mb) {
    const u32x4_t lo = *(const u32x4_t *)(st + alo + mb * 32 * C::AB);
    if constexpr (C::A_FP4) {
      an = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], 0, 0, 0, 0};
    } else {
      const u32x4_t hi = *(const u32x4_t *)(st + ahi + mb * 32 * C::AB);
      an = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
  };
  uint32_t sw_cur = 0, sa_cur[AM];
#pragma unroll
  for (int mb = 0; mb < AM; ++mb) sa_cur[mb] = 0;
  // Steps in runs of NS, one per stage, so that every stage address is a
  // constant offset (cur = t % NS is known in each copy of the body).
  for (int t0 = 0; t0 < T; t0 += NS) {
#pragma unroll
  for (int cur = 0; cur < NS; ++cur) {
    const int t = t0 + cur;
    if (t >= T) break;
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint8_t *const st = s_lds + cur * C::STAGE;
    const int nxt = cur == NS - 1 ? 0 : cur + 1;
    // Step t + 1 was published at this barrier and its stage is not
    // refilled before the next one.
    const uint8_t *const sx = s_lds + nxt * C::STAGE;
    if (t == 0) {
      read_w(st);
      read_s(st);
      read_a(st, 0);
    }
    const u32x4_t w0 = wn[0], w1 = wn[1];
    if ((t & 1) == 0) {
      sw_cur = sn;
#pragma unroll
      for (int mb = 0; mb < AM; ++mb) sa_cur[mb] = asn[mb];
    }
    // Bytes 2 f + j of the weight scale dword (opsel j), byte 2 f + h of a
    // row's scale dword, f = t & 1.
    const int sh = 16 * (t & 1);
    const int sb = sw_cur >> sh;
    const i32x8_t b0 = {(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3], 0, 0, 0, 0};
    const i32x8_t b1 = {(int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3], 0, 0, 0, 0};
#pragma unroll
    for (int mb = 0; mb < AM; ++mb) {
      const i32x8_t a = an;
      const int sa = (int)((sa_cur[mb] >> (sh + 8 * h)) & 0xFFu);
      __builtin_amdgcn_sched_barrier(0);
      if (mb + 1 < AM) {
        read_a(st, mb + 1);
      } else {
        read_a(sx, 0);
      }
      if (mb == 0) {
        read_w(sx);
        if ((t & 1) == 1) read_s(sx);
      }
      constexpr int AFMT = C::A_FP4 ? 4 : 0;  // A operand format: e2m1 or e4m3 (B: e2m1)
      acc[mb][0] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b0, acc[mb][0], AFMT, 4, 0, sa, 0, sb);
      acc[mb][1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b1, acc[mb][1], AFMT, 4, 0, sa, 1, sb);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  store_tile<AM, ACT, C::EP_STRIDE>(acc, (float *)(s_lds + cw * 32 * C::EP_STRIDE * 4), row0, rows, col0, N, out,
                                    out_f32, bias, ep.bias_bf16, ep.act);
}

// Producer dispatch on the lhs row groups that hold rows (NA) and on whether
// this producer also loads a part of the row scales.
template <class C, int NA = (C::A_GROUPS + C::NPROD - 1) / C::NPROD>
__device__ __forceinline__ void mx_produce(int na, bool asl, const uint8_t *lhs, const uint8_t *lsc,
                                           const int32_t *row_idx, int64_t lhs_rows, int64_t row0, int rows, int K,
                                           int T, int KB, const uint8_t *wexp, const uint8_t *sexp, int g0, int G,
                                           uint8_t *s_lds, int pw) {
  if constexpr (NA > 0) {
    if (na < NA) {
      mx_produce<C, NA - 1>(na, asl, lhs, lsc, row_idx, lhs_rows, row0, rows, K, T, KB, wexp, sexp, g0, G, s_lds, pw);
      return;
    }
  }
  if (asl)
    mx_producer<C, NA, true>(lhs, lsc, row_idx, lhs_rows, row0, rows, K, T, KB, wexp, sexp, g0, G, s_lds, pw);
  else
    mx_producer<C, NA, false>(lhs, lsc, row_idx, lhs_rows, row0, rows, K, T, KB, wexp, sexp, g0, G, s_lds, pw);
}

// A consumer whose row half holds no rows keeps the barrier count (T + 1).
__device__ __forceinline__ void mx_idle_consumer(int T) {
  for (int t = 0; t <= T; ++t) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
}

template <class C, bool ACT>
__global__ __launch_bounds__(C::THREADS) void gmm_mx_kernel(
    const uint8_t *__restrict__ lhs, const uint8_t *__restrict__ lsc, const int32_t *__restrict__ row_idx,
    int64_t lhs_rows, int64_t M, int K, const uint8_t *__restrict__ wpk, const uint8_t *__restrict__ spk,
    const int32_t *__restrict__ group_sizes, int num_groups, const int32_t *__restrict__ group_offset,
    int64_t e_local, int N, void *__restrict__ out, int out_f32, GmmEpilogue ep) {
  constexpr int CW = C::CONS, NP = C::NPROD, TMB = C::TMB, CMB = C::CMB;
  static_assert(C::STAGES * C::STAGE >= (kMaxGroups + TMB * kClsStride) * 4, "tile classes alias the stages");
  __shared__ __attribute__((aligned(1024))) uint8_t s_lds[C::STAGES * C::STAGE];
  __shared__ int s_info[kTileInfo];
  int *s_rowstart = (int *)s_lds;
  int *s_cls = s_rowstart + kMaxGroups;

  const int tid = threadIdx.x, wave = tid >> 6;
  const int go = group_offset ? group_offset[0] : 0;
  TileRef ref;
  if (!find_tile<TMB, 32, C::THREADS>(group_sizes, num_groups, go, e_local, M, (N + C::NT - 1) / C::NT, 0, 0, 0,
                                      s_rowstart, s_cls, s_info, ref))
    return;
  const int g = ref.g, nt = ref.nt, rows = ref.rows;
  const int64_t row0 = ref.row0;
  const int64_t e = g - go;
  const int T = K >> 6, KB = K >> 7, G = (N + 63) >> 6;
  const int g0 = nt * C::GT;
  if (wave >= CW) {
    const int pw = wave - CW;
    const uint8_t *const wexp = wpk + e * G * T * 2048;
    const uint8_t *const sexp = spk + e * G * KB * 256;
    // Row groups pw + NP i (< A_GROUPS) with RL (pw + NP i) < rows are loaded.
    int na = 0;
    for (int ga = pw; ga < C::A_GROUPS; ga += NP) na += C::RL * ga < rows ? 1 : 0;
    const bool asl = pw >= NP - C::AS_LOADS;
    mx_produce<C>(na, asl, lhs, lsc, row_idx, lhs_rows, row0, rows, K, T, KB, wexp, sexp, g0, G, s_lds, pw);
    return;
  }
  const int cg = wave % C::GT, rb = 32 * CMB * (wave / C::GT);
  const int rows_h = min(rows - rb, 32 * CMB);  // rows of this consumer's half
  if (rows_h <= 0) {
    mx_idle_consumer(T);
    return;
  }
  const int act_mb = (rows_h + 31) >> 5;
  const int64_t col0 = (int64_t)(g0 + cg) * 64;
  const void *const bias = expert_bias(ep, e, N);
  if (act_mb <= 1 || CMB == 1)
    mx_consumer<C, 1, ACT>(T, s_lds, wave, cg, rb, row0 + rb, rows_h, col0, N, out, out_f32, bias, ep);
  else if (act_mb == 2 || CMB == 2)
    mx_consumer<C, (CMB >= 2 ? 2 : 1), ACT>(T, s_lds, wave, cg, rb, row0 + rb, rows_h, col0, N, out, out_f32, bias,
                                            ep);
  else mx_consumer<C, CMB, ACT>(T, s_lds, wave, cg, rb, row0 + rb, rows_h, col0, N, out, out_f32, bias, ep);
}

// ---------------------------------------------------------------------------
// 128-deep steps: one scale dword per row and per weight-group lane covers a
// whole step (K-blocks 4 kb .. 4 kb + 3), so every step issues the same
// loads.  Per step and 96 x 512 tile: W 8 groups x 4 KiB (the two 64-deep
// halves of fp4.hip's layout, contiguous), A 96 rows x 128 bytes (chunk c of
// row r at physical chunk c ^ ((r >> 1) & 7)), AS 128 row dwords, S 8 x 256
// bytes.  Stage t is published at barrier t (one step ahead of the
// consumers' reads) and the stage of step t - 1 is refilled with step
// t + NS - 1.
// AF4: e2m1 lhs (MXFP4): 64 bytes per row and 128-deep step in four 16-byte
// chunks, chunk c of row r at physical chunk c ^ ((r >> 2) & 3) (the e4m3
// layout of the 64-deep kernel), 16 rows per 1 KiB load.
template <int MB, int CW, int NP, int NS, bool AF4 = false>
struct Mx128Cfg {
  static constexpr int CONS = CW, NPROD = NP, STAGES = NS;
  static constexpr bool A_FP4 = AF4;
  static constexpr int GT = CW;
  static constexpr int THREADS = 64 * (CW + NP);
  static constexpr int NT = 64 * GT;
  static constexpr int ROWS = 32 * MB;
  static constexpr int AB = AF4 ? 64 : 128;              // lhs bytes per row and step
  static constexpr int RL = 1024 / AB;                   // rows per 1 KiB lhs load
  static constexpr int W = 0;                            // group i: 4 KiB at W + 4096 i
  static constexpr int A = GT * 4096;                    // ROWS x AB bytes
  static constexpr int AS_LOADS = (ROWS + 63) / 64;
  static constexpr int AS = A + ROWS * AB;               // AS_LOADS x 256 bytes (dword per row)
  static constexpr int S = AS + AS_LOADS * 256;          // group i: 256 bytes at S + 256 i
  static constexpr int STAGE = S + GT * 256;
  static constexpr int A_GROUPS = ROWS / RL;             // 1 KiB lhs loads per step
  static constexpr int A_LOADS = (A_GROUPS + NP - 1) / NP;  // most lhs loads of one producer (groups pw + NP i)
  static constexpr int G_LOADS = GT / NP;
  static constexpr int EP_STRIDE = 72;
  static_assert(A_GROUPS * RL == ROWS && G_LOADS * NP == GT, "load split");
  static_assert(AS_LOADS <= NP && NS >= 2, "config");
  static_assert(CW * 32 * EP_STRIDE * 4 <= NS * STAGE, "epilogue staging fits the stages");
};

template <class C>
__device__ __forceinline__ int mx128_swz(int r) { return C::A_FP4 ? ((r >> 2) & 3) : ((r >> 1) & 7); }

template <class C, int NA, bool ASL>
__device__ __forceinline__ void mx128_producer(const uint8_t *__restrict__ lhs, const uint8_t *__restrict__ lsc,
                                               const int32_t *__restrict__ row_idx, int64_t lhs_rows, int64_t row0,
                                               int rows, int K, int T, const uint8_t *__restrict__ wexp,
                                               const uint8_t *__restrict__ sexp, int g0, int G, uint8_t *s_lds,
                                               int pw) {
  constexpr int NP = C::NPROD, NS = C::STAGES;
  constexpr int LOADS = NA + 5 * C::G_LOADS + (ASL ? 1 : 0);
  constexpr int PENDING = LOADS * (NS - 2);  // steps t + 1 .. t + NS - 2 may be pending at barrier t
  static_assert(PENDING < 64, "vmcnt range");
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = NA; i < C::A_LOADS; ++i) {
    const int ga = pw + NP * i;
    if (ga < C::A_GROUPS) {
#pragma unroll
      for (int st = 0; st < NS; ++st)
        *(u32x4_t *)(s_lds + st * C::STAGE + C::A + ga * 1024 + lane * 16) = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
  const int KS = K / kMxBlock;
  auto src_row = [&](int r) -> int64_t {
    const int rs = r < rows ? r : rows - 1;
    return row_idx ? gather_index(row_idx[row0 + rs], lhs_rows) : row0 + rs;
  };
  // lhs load i: rows RL (pw + NP i) .. + RL - 1; lane l fills physical chunk
  // l % LPR of row + l / LPR with the logical chunk of the swizzle.
  constexpr int LPR = C::AB / 16;
  const int64_t KR = C::A_FP4 ? K / 2 : K;  // lhs bytes per row
  uint32_t aoff[NA > 0 ? NA : 1];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int r = C::RL * (pw + NP * i) + lane / LPR;
    aoff[i] = (uint32_t)(src_row(r) * KR) + (uint32_t)(((lane % LPR) ^ mx128_swz<C>(r)) << 4);
  }
  const int aspart = pw - (NP - C::AS_LOADS);
  const uint32_t asoff = ASL ? (uint32_t)(src_row(64 * aspart + lane) * KS) : 0u;
  const uint8_t *wsrc[C::G_LOADS];
  const uint8_t *ssrc[C::G_LOADS];
#pragma unroll
  for (int c = 0; c < C::G_LOADS; ++c) {
    const int g = min(g0 + pw + NP * c, G - 1);
    wsrc[c] = wexp + (int64_t)g * T * 4096 + lane * 16;
    ssrc[c] = sexp + (int64_t)g * T * 256 + lane * 4;
  }
  auto issue = [&](int stage, int t) {
    uint8_t *const st = s_lds + stage * C::STAGE;
    const uint8_t *const a = lhs + (int64_t)t * C::AB;
#pragma unroll
    for (int i = 0; i < NA; ++i)
      __builtin_amdgcn_global_load_lds((const void *)(a + aoff[i]),
                                       (lds_void_t *)(st + C::A + (pw + NP * i) * 1024), 16, 0, 0);
#pragma unroll
    for (int c = 0; c < C::G_LOADS; ++c) {
      const int gi = pw + NP * c;
      const uint8_t *const w = wsrc[c] + (int64_t)t * 4096;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        __builtin_amdgcn_global_load_lds((const void *)(w + 1024 * q),
                                         (lds_void_t *)(st + C::W + gi * 4096 + 1024 * q), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void *)(ssrc[c] + (int64_t)t * 256),
                                       (lds_void_t *)(st + C::S + gi * 256), 4, 0, 0);
    }
    if (ASL)
      __builtin_amdgcn_global_load_lds((const void *)(lsc + asoff + t * 4),
                                       (lds_void_t *)(st + C::AS + aspart * 256), 4, 0, 0);
  };
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) issue(t, min(t, T - 1));
  int refill = NS - 1;
  for (int t = 0; t < T; ++t) {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(PENDING));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(refill, min(t + NS - 1, T - 1));
    refill = refill == NS - 1 ? 0 : refill + 1;
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
}

template <class C, int AM, bool ACT>
__device__ __forceinline__ void mx128_consumer(int T, uint8_t *s_lds, int cw, int64_t row0, int rows, int64_t col0,
                                               int N, void *__restrict__ out, int out_f32, const void *bias,
                                            const GmmEpilogue &ep) {
  constexpr int NS = C::STAGES;
  const int lane = threadIdx.x & 63, c32 = lane & 31, h = lane >> 5;
  f32x16_t acc[AM][2];
#pragma unroll
  for (int mb = 0; mb < AM; ++mb)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][j][r] = 0.0f;
  const int woff = C::W + cw * 4096 + lane * 16;
  const int soff = C::S + cw * 256 + lane * 4;
  const int sw = mx128_swz<C>(c32);  // rows mb * 32 + c32 share it
  const int arow = C::A + c32 * C::AB;
  u32x4_t wa[2], wb[2];
  i32x8_t an;
  // A fragment of substep f (k = 64 f .. + 63): e4m3 chunks 4 f + h and
  // 4 f + 2 + h; e2m1 chunk 2 f + h (k = 64 f + 32 h .. + 31).
  auto read_a = [&](const uint8_t *st, int f, int mb) {
    if constexpr (C::A_FP4) {
      const u32x4_t lo = *(const u32x4_t *)(st + arow + mb * 32 * C::AB + (((2 * f + h) ^ sw) << 4));
      an = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], 0, 0, 0, 0};
    } else {
      const u32x4_t lo = *(const u32x4_t *)(st + arow + mb * 32 * C::AB + (((4 * f + h) ^ sw) << 4));
      const u32x4_t hi = *(const u32x4_t *)(st + arow + mb * 32 * C::AB + (((4 * f + 2 + h) ^ sw) << 4));
      an = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
  };
  // Steps in runs of NS, one per stage, so that every stage address is a
  // constant offset (cur = t % NS is known in each copy of the body).
  for (int t0 = 0; t0 < T; t0 += NS) {
#pragma unroll
  for (int cur = 0; cur < NS; ++cur) {
    if (t0 + cur >= T) break;
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint8_t *const st = s_lds + cur * C::STAGE;
    wa[0] = *(const u32x4_t *)(st + woff);
    wa[1] = *(const u32x4_t *)(st + woff + 1024);
    const uint32_t sd = *(const uint32_t *)(st + soff);
    uint32_t sa[AM];
#pragma unroll
    for (int mb = 0; mb < AM; ++mb) sa[mb] = *(const uint32_t *)(st + C::AS + (mb * 32 + c32) * 4);
    read_a(st, 0, 0);
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const u32x4_t w0 = f == 0 ? wa[0] : wb[0], w1 = f == 0 ? wa[1] : wb[1];
      const i32x8_t b0 = {(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3], 0, 0, 0, 0};
      const i32x8_t b1 = {(int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3], 0, 0, 0, 0};
      const int sb = (int)(sd >> (16 * f));
#pragma unroll
      for (int mb = 0; mb < AM; ++mb) {
        const i32x8_t a = an;
        const int sa_l = (int)((sa[mb] >> (16 * f + 8 * h)) & 0xFFu);
        __builtin_amdgcn_sched_barrier(0);
        if (mb + 1 < AM) read_a(st, f, mb + 1);
        else if (f == 0) read_a(st, 1, 0);
        if (f == 0 && mb == 0) {
          wb[0] = *(const u32x4_t *)(st + woff + 2048);
          wb[1] = *(const u32x4_t *)(st + woff + 3072);
        }
        constexpr int AFMT = C::A_FP4 ? 4 : 0;  // A operand format: e2m1 or e4m3 (B: e2m1)
        acc[mb][0] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b0, acc[mb][0], AFMT, 4, 0, sa_l, 0, sb);
        acc[mb][1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b1, acc[mb][1], AFMT, 4, 0, sa_l, 1, sb);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  store_tile<AM, ACT, C::EP_STRIDE>(acc, (float *)(s_lds + cw * 32 * C::EP_STRIDE * 4), row0, rows, col0, N, out,
                                    out_f32, bias, ep.bias_bf16, ep.act);
}

template <class C, int MB, bool ACT>
__global__ __launch_bounds__(C::THREADS) void gmm_mx128_kernel(
    const uint8_t *__restrict__ lhs, const uint8_t *__restrict__ lsc, const int32_t *__restrict__ row_idx,
    int64_t lhs_rows, int64_t M, int K, const uint8_t *__restrict__ wpk, const uint8_t *__restrict__ spk,
    const int32_t *__restrict__ group_sizes, int num_groups, const int32_t *__restrict__ group_offset,
    int64_t e_local, int N, void *__restrict__ out, int out_f32, GmmEpilogue ep) {
  constexpr int CW = C::CONS, NP = C::NPROD;
  static_assert(C::STAGES * C::STAGE >= (kMaxGroups + MB * kClsStride) * 4, "tile classes alias the stages");
  __shared__ __attribute__((aligned(1024))) uint8_t s_lds[C::STAGES * C::STAGE];
  __shared__ int s_info[kTileInfo];
  int *s_rowstart = (int *)s_lds;
  int *s_cls = s_rowstart + kMaxGroups;
  const int tid = threadIdx.x, wave = tid >> 6;
  const int go = group_offset ? group_offset[0] : 0;
  TileRef ref;
  if (!find_tile<MB, 32, C::THREADS>(group_sizes, num_groups, go, e_local, M, (N + C::NT - 1) / C::NT, 0, 0, 0,
                                 s_rowstart, s_cls, s_info, ref))
    return;
  const int g = ref.g, nt = ref.nt, rows = ref.rows;
  const int64_t row0 = ref.row0;
  const int64_t e = g - go;
  const int T = K >> 7, G = (N + 63) >> 6;
  const int g0 = nt * C::GT;
  if (wave >= CW) {
    const int pw = wave - CW;
    const uint8_t *const wexp = wpk + e * G * T * 4096;
    const uint8_t *const sexp = spk + e * G * T * 256;
    // Row groups pw + NP i (< A_GROUPS) with RL (pw + NP i) < rows are loaded.
    int na = 0;
    for (int ga = pw; ga < C::A_GROUPS; ga += NP) na += C::RL * ga < rows ? 1 : 0;
    const bool asl = pw >= NP - C::AS_LOADS;
    auto run = [&](auto na_c, auto asl_c) {
      mx128_producer<C, (decltype(na_c)::value < C::A_LOADS ? decltype(na_c)::value : C::A_LOADS),
                     decltype(asl_c)::value != 0>(lhs, lsc, row_idx, lhs_rows, row0, rows, K, T, wexp, sexp, g0, G,
                                                  s_lds, pw);
    };
    static_assert(C::A_LOADS <= 3, "at most three lhs row groups per producer");
    if (asl) {
      if (na >= 3) run(IntC<3>{}, IntC<1>{});
      else if (na == 2) run(IntC<2>{}, IntC<1>{});
      else if (na == 1) run(IntC<1>{}, IntC<1>{});
      else run(IntC<0>{}, IntC<1>{});
    } else {
      if (na >= 3) run(IntC<3>{}, IntC<0>{});
      else if (na == 2) run(IntC<2>{}, IntC<0>{});
      else if (na == 1) run(IntC<1>{}, IntC<0>{});
      else run(IntC<0>{}, IntC<0>{});
    }
    return;
  }
  const int act_mb = (rows + 31) >> 5;
  const int64_t col0 = (int64_t)(g0 + wave) * 64;
  const void *const bias = expert_bias(ep, e, N);
  if (act_mb <= 1 || MB == 1) mx128_consumer<C, 1, ACT>(T, s_lds, wave, row0, rows, col0, N, out, out_f32, bias, ep);
  else if (act_mb == 2 || MB == 2) mx128_consumer<C, (MB >= 2 ? 2 : 1), ACT>(T, s_lds, wave, row0, rows, col0, N, out, out_f32, bias, ep);
  else mx128_consumer<C, MB, ACT>(T, s_lds, wave, row0, rows, col0, N, out, out_f32, bias, ep);
}

template <class C, int MB, bool ACT, bool STEP128>
static int launch_mx(const uint8_t *lhs, const uint8_t *lsc, const int32_t *row_idx, int64_t lhs_rows, int64_t M,
                     int64_t K, const uint8_t *w, const uint8_t *s, const int32_t *gs, int ng, const int32_t *go,
                     int64_t e_local, int64_t N, void *out, int out_f32, const GmmEpilogue &ep, hipStream_t st) {
  constexpr int MT = 32 * MB, NT = C::NT;
  const int64_t n_tiles = (N + NT - 1) / NT;
  const int64_t max_tiles = ((M + MT - 1) / MT + e_local) * n_tiles;
  const int64_t grid = ((max_tiles + 7) / 8 + MB) * 8;
  DWM_UNSUPPORTED_IF(grid > (1ll << 31) - 1, "gmm_fp4_mx: too many tiles (%lld)", (long long)grid);
  if constexpr (STEP128)
    hipLaunchKernelGGL((gmm_mx128_kernel<C, MB, ACT>), dim3((unsigned)grid), dim3(C::THREADS), 0, st, lhs, lsc,
                       row_idx, lhs_rows, M, (int)K, w, s, gs, ng, go, e_local, (int)N, out, out_f32, ep);
  else
    hipLaunchKernelGGL((gmm_mx_kernel<C, ACT>), dim3((unsigned)grid), dim3(C::THREADS), 0, st, lhs, lsc, row_idx,
                       lhs_rows, M, (int)K, w, s, gs, ng, go, e_local, (int)N, out, out_f32, ep);
  return launch_status("gmm_fp4_mx");
}

// The MX grouped matmul (arguments checked by the caller).
int launch_gmm_mx(const uint8_t *lhs, const uint8_t *lhs_scale, const int32_t *row_idx, int64_t lhs_rows, int64_t M,
                  int64_t K, const uint8_t *weight, const uint8_t *scale, const int32_t *group_sizes, int num_groups,
                  const int32_t *group_offset, int64_t E_local, int64_t N, void *out, int out_f32, bool gated,
                  const GmmEpilogue &ep, hipStream_t st, bool lhs_fp4) {
  // 96-row x 512-column tiles, 8 consumer + 4 producer waves.  64-deep K
  // steps in a five-stage ring (two published per barrier, two in flight),
  // or 128-deep steps in a three-stage ring (one published, one in flight).
  // Below K = 4096, groups of 97 .. 192 rows on average run 192 x 256
  // tiles (two stacked row halves), so their weights are read once:
  // decode_down (~128 rows per group) 111 -> 106 us, measured against the
  // 96 x 512 tiles; seven stages in place of five were slower (110 us).
  // Larger groups read their weights once per row tile either way.
  using C64 = MxCfg<3, 8, 4, 5>;
  using C64H = MxCfg<3, 8, 4, 5, 2>;
  using C128 = Mx128Cfg<3, 8, 4, 3>;
  // MXFP4 lhs: the same kernels with e2m1 A operands.
  using F64 = MxCfg<3, 8, 4, 5, 1, true>;
  using F64H = MxCfg<3, 8, 4, 5, 2, true>;
  using F128 = Mx128Cfg<3, 8, 4, 3, true>;
  const bool deep = K >= kMx128MinK;
  const bool halves = !deep && M > 96 * E_local && M <= 192 * E_local;
#define DWM_MX(CFG, TMB, ACT, DEEP)                                                                                \
  launch_mx<CFG, TMB, ACT, DEEP>(lhs, lhs_scale, row_idx, lhs_rows, M, K, weight, scale, group_sizes, num_groups, \
                                 group_offset, E_local, N, out, out_f32, ep, st)
  if (lhs_fp4) {
    if (gated)
      return deep ? DWM_MX(F128, 3, true, true) : halves ? DWM_MX(F64H, 6, true, false) : DWM_MX(F64, 3, true, false);
    return deep ? DWM_MX(F128, 3, false, true) : halves ? DWM_MX(F64H, 6, false, false) : DWM_MX(F64, 3, false, false);
  }
  if (gated)
    return deep ? DWM_MX(C128, 3, true, true) : halves ? DWM_MX(C64H, 6, true, false) : DWM_MX(C64, 3, true, false);
  return deep ? DWM_MX(C128, 3, false, true) : halves ? DWM_MX(C64H, 6, false, false) : DWM_MX(C64, 3, false, false);
#undef DWM_MX
}

}  // namespace dwm

using namespace dwm;

extern "C" int dwm_mx_quant_e2m1(const uint16_t *x, int64_t rows, int64_t K, uint8_t *codes, uint8_t *scales,
                                 void *stream) {
  clear_error();
  DWM_CHECK_ARG(rows >= 0 && K > 0, "mx_quant_e2m1: bad sizes rows=%lld K=%lld", (long long)rows, (long long)K);
  DWM_UNSUPPORTED_IF(K % kMxBlock != 0, "mx_quant_e2m1: K %% 32 == 0 required (K=%lld)", (long long)K);
  if (rows == 0) return DWM_OK;
  DWM_CHECK_ARG(x && codes && scales, "mx_quant_e2m1: null pointer");
  DWM_CHECK_ARG((uintptr_t)x % 16 == 0 && (uintptr_t)codes % 4 == 0,
                "mx_quant_e2m1: x must be 16-byte and codes 4-byte aligned");
  const int64_t n8 = rows * K / 8;
  int64_t blocks = (n8 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(mx_quant_e2m1_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), x, n8, codes,
                     scales);
  return launch_status("mx_quant_e2m1");
}

extern "C" int dwm_mx_quant_e4m3(const uint16_t *x, int64_t rows, int64_t K, uint8_t *codes, uint8_t *scales,
                                 void *stream) {
  clear_error();
  DWM_CHECK_ARG(rows >= 0 && K > 0, "mx_quant_e4m3: bad sizes rows=%lld K=%lld", (long long)rows, (long long)K);
  DWM_UNSUPPORTED_IF(K % kMxBlock != 0, "mx_quant_e4m3: K %% 32 == 0 required (K=%lld)", (long long)K);
  if (rows == 0) return DWM_OK;
  DWM_CHECK_ARG(x && codes && scales, "mx_quant_e4m3: null pointer");
  DWM_CHECK_ARG((uintptr_t)x % 16 == 0 && (uintptr_t)codes % 8 == 0,
                "mx_quant_e4m3: x must be 16-byte and codes 8-byte aligned");
  const int64_t n8 = rows * K / 8;
  int64_t blocks = (n8 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(mx_quant_e4m3_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), x, n8, codes,
                     scales);
  return launch_status("mx_quant_e4m3");
}

