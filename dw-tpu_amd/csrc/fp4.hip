// FP4 weight formats: e2m1 -> gmm_v2 codes, the decode test hook, and the
// load-time prepack into the layout the grouped-matmul kernel streams.
//
// Prepacked weight layout: per expert e, 64-column group g (G = ceil(N/64)
// groups; columns past N are padding with zero codes), 64-deep K step t
// (T = K/64) and 32-column half j, one 1 KiB block
//   weight[(((e * G + g) * T + t) * 2 + j) * 1024 + lane * 16 + i]
//   lane = c + 32*h: column 64*g + 32*j + c; byte i holds the e2m1 nibbles of
//   k = 64*t + 32*h + 2*i (low) and k + 1 (high).
// Lane l's 16 bytes are the 32 consecutive K values of its column in one
// 32-element scale block, which is the bf16 MFMA 32x32x16 B-operand order the
// kernel decodes into (dword s of the lane feeds MFMA step s of the K step).
// Prepacked scales: per (e, g, 128-deep step kb) 256 bytes
//   scale[((e * G + g) * (K/128) + kb) * 256 + lane * 4 + 2*f + j]
//   = e8m0 code of column 64*g + 32*j + c, K-block 4*kb + 2*f + h
// (f: which 64-deep half of the 128-deep step), so one dword per lane holds
// every scale a 64-column group needs for two K steps.
#include "common.h"

namespace dwm {

// gmm_v2 code (int4 q in a nibble) -> canonical e2m1 nibble; q = -8 has no
// e2m1 value and sets *bad.
__device__ __forceinline__ uint32_t code_to_e2m1(uint32_t c, bool *bad) {
  c &= 0xFu;
  if (c == 8u) { *bad = true; return 0u; }
  return (c & 8u) ? (8u | ((16u - c) & 7u)) : c;
}

// e2m1 nibble -> canonical nibble (-0 -> +0, as e2m1_to_codes maps it).
__device__ __forceinline__ uint32_t canon_e2m1(uint32_t c) {
  c &= 0xFu;
  return c == 8u ? 0u : c;
}

__device__ __forceinline__ uint32_t e2m1_to_code_nib(uint32_t c) {
  c &= 0xFu;
  uint32_t m = c & 7u;
  return (c & 8u) ? ((16u - m) & 0xFu) : m;
}

// Scale element -> e8m0 code; sets *bad unless it is +0.0 or a normal power
// of two (the lossless set of e8m0_encode).
__device__ __forceinline__ uint32_t scale_to_code(const void *scale, int dtype, int64_t idx,
                                                  bool *bad) {
  if (dtype == DWM_U8) {
    uint32_t c = ((const uint8_t *)scale)[idx];
    if (c == 255u) *bad = true;
    return c;
  }
  uint32_t bits;
  if (dtype == DWM_F32) bits = ((const uint32_t *)scale)[idx];
  else bits = (uint32_t)((const uint16_t *)scale)[idx] << 16;
  uint32_t e = bits >> 23;
  if ((bits & 0x807FFFFFu) != 0u || e == 255u) *bad = true;
  return e & 0xFFu;
}

__global__ void e2m1_to_codes_kernel(const uint8_t *in, uint8_t *out, int64_t nbytes) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < nbytes; i += stride) {
    uint32_t b = in[i];
    out[i] = (uint8_t)(e2m1_to_code_nib(b) | (e2m1_to_code_nib(b >> 4) << 4));
  }
}

// One thread per pair of values (one input byte).
__global__ void fp4_decode_kernel(const uint8_t *packed, int format, int64_t nbytes,
                                  const uint8_t *scales, uint32_t *out, int32_t *flags) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nbytes) return;
  uint32_t b = packed[i];
  uint32_t n0 = b & 0xFu, n1 = b >> 4;
  bool bad = false;
  uint32_t c0 = format == DWM_FP4_CODES ? code_to_e2m1(n0, &bad) : canon_e2m1(n0);
  uint32_t c1 = format == DWM_FP4_CODES ? code_to_e2m1(n1, &bad) : canon_e2m1(n1);
  uint32_t sc = scales ? scales[(2 * i) >> 5] : 127u;
  uint32_t r;
  if (sc == 0u) {
    // decode(q) * bf16(+0.0): +-0 with the sign of the value.
    r = ((c0 & 8u) ? 0x8000u : 0u) | ((c1 & 8u) ? 0x80000000u : 0u);
  } else if (sc == 255u) {
    r = 0x7FC07FC0u;
    atomicOr(flags, 1);
  } else {
    r = cvt_fp4x2_bf16<0>(c0 | (c1 << 4), e8m0_to_f32(sc));
  }
  if (bad) {
    // q = -8: decode_codes gives -8 (= 2q - (clip(q,-6,6) + clip(q,-4,4)/2)),
    // which the e2m1 converter cannot produce; computed directly.
    float s = scales ? e8m0_to_f32(sc) : 1.0f;
    uint32_t hi = r >> 16, lo = r & 0xFFFFu;
    if ((n0 & 0xFu) == 8u) lo = f32_to_bf16_bits(-8.0f * s);
    if ((n1 & 0xFu) == 8u) hi = f32_to_bf16_bits(-8.0f * s);
    r = lo | (hi << 16);
    atomicOr(flags, 2);
  }
  out[i] = r;
}

// One thread per (e, g, kb, lane): the four 16-byte pieces of lane `lane` in
// the two 64-deep steps of 128-deep step kb (both halves j) and its scale word.
// With gate_up, packed column 64 g + 32 j + c takes source column
// j * N/2 + 32 g + c: half 0 of every group is 32 gate columns and half 1 the
// matching up columns of a [w1 | w3] weight, so the kernel's fused activation
// finds both in one wave.
// transposed: rhs is [E, N, K/2] (two K values per byte, low nibble = even
// k) instead of [E, K, N/2].
__global__ void gmm_fp4_prepack_kernel(const uint8_t *rhs, int format, const void *scale,
                                       int scale_dtype, int64_t E, int64_t K, int64_t N,
                                       uint8_t *wout, uint8_t *sout, int32_t *flags, int gate_up,
                                       int transposed) {
  const int64_t G = (N + 63) / 64, KB = K / 128, T = K / 64;
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = E * G * KB * 64;
  if (t >= total) return;
  const int lane = (int)(t & 63);
  int64_t r = t >> 6;
  const int64_t kb = r % KB;
  r /= KB;
  const int64_t g = r % G;
  const int64_t e = r / G;
  const int c = lane & 31, h = lane >> 5;
  const int64_t half_n = N / 2;
  bool bad_scale = false, bad_code = false;
  uint32_t sword = 0;
#pragma unroll
  for (int f = 0; f < 2; ++f) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t np = g * 64 + 32 * j + c;  // packed column
      const int64_t n = gate_up ? j * (N / 2) + 32 * g + c : np;
      const int64_t k0 = kb * 128 + 64 * f + 32 * h;
      uint32_t code = 127u;
      uint32_t words[4] = {0u, 0u, 0u, 0u};
      if (np < N) {
        code = scale_to_code(scale, scale_dtype, (e * (K / 32) + (k0 >> 5)) * N + n, &bad_scale);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t word = 0;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int64_t k = k0 + 8 * w + i;
            const uint32_t byte = transposed ? rhs[(e * N + n) * (K / 2) + (k >> 1)]
                                             : rhs[(e * K + k) * half_n + (n >> 1)];
            uint32_t nib = ((transposed ? k : n) & 1) ? (byte >> 4) : (byte & 0xFu);
            nib = format == DWM_FP4_CODES ? code_to_e2m1(nib, &bad_code) : canon_e2m1(nib);
            if (code == 0u) nib &= 8u;  // zero scale: keep only the sign -> +-0
            word |= nib << (4 * i);
          }
          words[w] = word;
        }
        if (code == 0u) code = 127u;
      }
      sword |= (code & 0xFFu) << (8 * (2 * f + j));
      const u32x4_t v = {words[0], words[1], words[2], words[3]};
      *(u32x4_t *)(wout + (((e * G + g) * T + 2 * kb + f) * 2 + j) * 1024 + lane * 16) = v;
    }
  }
  *(uint32_t *)(sout + ((e * G + g) * KB + kb) * 256 + lane * 4) = sword;
  if (bad_scale) atomicOr(flags, 1);
  if (bad_code) atomicOr(flags, 2);
}

}  // namespace dwm

using namespace dwm;

extern "C" int dwm_e2m1_to_codes(const uint8_t *e2m1, uint8_t *codes, int64_t nbytes,
                                 void *stream) {
  clear_error();
  DWM_CHECK_ARG(nbytes >= 0, "e2m1_to_codes: nbytes < 0");
  if (nbytes == 0) return DWM_OK;
  DWM_CHECK_ARG(e2m1 && codes, "e2m1_to_codes: null pointer");
  int64_t blocks = (nbytes + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(e2m1_to_codes_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     e2m1, codes, nbytes);
  return launch_status("e2m1_to_codes");
}

extern "C" int dwm_fp4_decode(const uint8_t *packed, int format, int64_t n, const uint8_t *scales,
                              uint16_t *out_bf16, int32_t *flags, void *stream) {
  clear_error();
  DWM_CHECK_ARG(n >= 0 && n % 2 == 0, "fp4_decode: n must be even and >= 0 (got %lld)", (long long)n);
  DWM_CHECK_ARG(format == DWM_FP4_E2M1 || format == DWM_FP4_CODES, "fp4_decode: bad format %d", format);
  if (n == 0) return DWM_OK;
  DWM_CHECK_ARG(packed && out_bf16 && flags, "fp4_decode: null pointer");
  int64_t nbytes = n / 2;
  int64_t blocks = (nbytes + 255) / 256;
  DWM_CHECK_ARG(blocks < (1ll << 31), "fp4_decode: n too large");
  hipLaunchKernelGGL(fp4_decode_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     packed, format, nbytes, scales, (uint32_t *)out_bf16, flags);
  return launch_status("fp4_decode");
}

extern "C" int dwm_gmm_fp4_prepack_size(int64_t E, int64_t K, int64_t N, int64_t *weight_bytes,
                                        int64_t *scale_bytes) {
  clear_error();
  DWM_CHECK_ARG(E >= 0 && K > 0 && N > 0, "gmm_fp4_prepack_size: bad sizes E=%lld K=%lld N=%lld",
                (long long)E, (long long)K, (long long)N);
  DWM_UNSUPPORTED_IF(K % 128 != 0 || N % 16 != 0,
                     "gmm_fp4: K %% 128 == 0 and N %% 16 == 0 required (K=%lld N=%lld)",
                     (long long)K, (long long)N);
  DWM_CHECK_ARG(weight_bytes && scale_bytes, "gmm_fp4_prepack_size: null output pointer");
  const int64_t G = (N + 63) / 64;
  *weight_bytes = E * G * 64 * K / 2;
  *scale_bytes = E * G * (K / 128) * 256;
  return DWM_OK;
}

static int gmm_fp4_prepack_impl(const uint8_t *rhs, int format, const void *scale, int scale_dtype, int64_t E,
                                int64_t K, int64_t N, uint8_t *weight_out, uint8_t *scale_out, int32_t *flags,
                                int gate_up, int transposed, void *stream) {
  int64_t wb, sb;
  int st = dwm_gmm_fp4_prepack_size(E, K, N, &wb, &sb);
  if (st != DWM_OK) return st;
  DWM_CHECK_ARG(format == DWM_FP4_E2M1 || format == DWM_FP4_CODES, "gmm_fp4_prepack: bad format %d", format);
  DWM_CHECK_ARG(scale_dtype == DWM_U8 || scale_dtype == DWM_F32 || scale_dtype == DWM_BF16,
                "gmm_fp4_prepack: bad scale dtype %d", scale_dtype);
  DWM_UNSUPPORTED_IF(gate_up && N % 64 != 0, "gmm_fp4_prepack_gate_up: N %% 64 == 0 required (N=%lld)",
                     (long long)N);
  if (E == 0) return DWM_OK;
  DWM_CHECK_ARG(rhs && scale && weight_out && scale_out && flags, "gmm_fp4_prepack: null pointer");
  const int64_t total = E * ((N + 63) / 64) * (K / 128) * 64;
  const int64_t blocks = (total + 255) / 256;
  DWM_CHECK_ARG(blocks < (1ll << 31), "gmm_fp4_prepack: too large");
  hipLaunchKernelGGL(gmm_fp4_prepack_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), rhs, format,
                     scale, scale_dtype, E, K, N, weight_out, scale_out, flags, gate_up, transposed);
  return launch_status("gmm_fp4_prepack");
}

extern "C" int dwm_gmm_fp4_prepack(const uint8_t *rhs, int format, const void *scale,
                                   int scale_dtype, int64_t E, int64_t K, int64_t N,
                                   uint8_t *weight_out, uint8_t *scale_out, int32_t *flags,
                                   void *stream) {
  return gmm_fp4_prepack_impl(rhs, format, scale, scale_dtype, E, K, N, weight_out, scale_out, flags, 0, 0, stream);
}

extern "C" int dwm_gmm_fp4_prepack_gate_up(const uint8_t *rhs, int format, const void *scale, int scale_dtype,
                                           int64_t E, int64_t K, int64_t N, uint8_t *weight_out,
                                           uint8_t *scale_out, int32_t *flags, void *stream) {
  return gmm_fp4_prepack_impl(rhs, format, scale, scale_dtype, E, K, N, weight_out, scale_out, flags, 1, 0, stream);
}

extern "C" int dwm_gmm_fp4_prepack_transposed(const uint8_t *rhs, int format, const void *scale, int scale_dtype,
                                              int64_t E, int64_t K, int64_t N, int gate_up, uint8_t *weight_out,
                                              uint8_t *scale_out, int32_t *flags, void *stream) {
  return gmm_fp4_prepack_impl(rhs, format, scale, scale_dtype, E, K, N, weight_out, scale_out, flags,
                              gate_up ? 1 : 0, 1, stream);
}
