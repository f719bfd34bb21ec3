// Shared helpers of the gfx950 kernels and the C ABI: error reporting,
// argument checks, bf16 rounding, fp4 decode and wavefront scans.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/dwtpu_moe.h"

namespace dwm {

// ---- host-side error reporting -------------------------------------------

void set_error(const char *fmt, ...);
void clear_error();

#define DWM_CHECK_ARG(cond, ...)        \
  do {                                  \
    if (!(cond)) {                      \
      ::dwm::set_error(__VA_ARGS__);    \
      return DWM_ERR_INVALID;           \
    }                                   \
  } while (0)

#define DWM_UNSUPPORTED_IF(cond, ...)   \
  do {                                  \
    if (cond) {                         \
      ::dwm::set_error(__VA_ARGS__);    \
      return DWM_ERR_UNSUPPORTED;       \
    }                                   \
  } while (0)

// Reports the launch status of the kernels just enqueued.
int launch_status(const char *what);

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// ---- device helpers --------------------------------------------------------

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

// float -> bf16 bits, round to nearest even (f32 denormals kept); a NaN keeps
// its sign and top payload bits and is made quiet: bits (u >> 16) | 0x40.
// gfx950's v_cvt_pk_bf16_f32 (what the __bf16 conversion compiles to) gives
// exactly these bits for every one of the 2^32 inputs, in either half of its
// packed result, so no software rounding is needed.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two floats -> packed bf16 bits (lo in bits 0..15), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  const bf16x2_t p = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, p);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __builtin_bit_cast(float, b << 16);
}

// Two e2m1 nibbles of byte `SEL` of `src` -> packed bf16x2 (low nibble in the
// low half), each multiplied by 2^(e-127) where e is the exponent field of
// `scale`.  The result is bit-cast to u32 at once: extracting bf16 vector
// elements of the builtin's result directly miscompiles (both halves come
// out equal to the low one).
template <int SEL>
__device__ __forceinline__ uint32_t cvt_fp4x2_bf16(uint32_t src, float scale) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(src, scale, SEL));
}

typedef __attribute__((ext_vector_type(2))) short i16x2_t;

// Four f32 of magnitude <= 448 -> e4m3 codes, round to nearest even (the
// converter with unit scale; larger magnitudes never reach it here).
__device__ __forceinline__ uint32_t f32x4_e4m3(const float *v) {
  i16x2_t r = {0, 0};
  r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, v[0], v[1], 1.0f, false);
  r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, v[2], v[3], 1.0f, true);
  return __builtin_bit_cast(uint32_t, r);
}

// e8m0 code -> the f32 with that exponent field (2^(c-127) for 1 <= c <= 254).
__device__ __forceinline__ float e8m0_to_f32(uint32_t code) {
  return __builtin_bit_cast(float, (code & 0xFFu) << 23);
}

// LDS pointer type of the direct global -> LDS loads (global_load_lds).
typedef __attribute__((address_space(3))) void lds_void_t;

// Raw buffer resource over [base, base + bytes) (gfx9 descriptor word 3:
// 32-bit data format, no swizzle) for buffer_load ... lds: the address is a
// scalar base plus a per-lane 32-bit offset plus a scalar offset, so a load
// stream that advances by a uniform stride needs no vector arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// SIZE bytes per lane from rsrc at voffset + soffset into LDS at lds + SIZE * lane
// (SIZE must be a literal: the builtin takes it as an immediate).  The host
// pass of a HIP compile also instantiates kernel templates, to emit their
// launch stubs; it rejects this target builtin inside them without a
// diagnostic and drops the stub, so there the call is a no-op.
#if defined(__HIP_DEVICE_COMPILE__)
#define buffer_load_lds(SIZE, rsrc, lds, voffset, soffset) \
  __builtin_amdgcn_raw_ptr_buffer_load_lds((rsrc), (lds_void_t *)(lds), SIZE, (voffset), (soffset), 0, 0)
#else
#define buffer_load_lds(SIZE, rsrc, lds, voffset, soffset) ((void)(rsrc), (void)(lds), (void)(voffset), (void)(soffset))
#endif

// s_waitcnt immediate (gfx9 encoding): vmcnt <= vm, lgkmcnt == 0, expcnt untouched.
__host__ __device__ constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4); }

// JAX gather index semantics: wrap a negative index once, then clamp.
__device__ __forceinline__ int64_t gather_index(int64_t i, int64_t n) {
  if (i < 0) i += n;
  if (i < 0) i = 0;
  if (i >= n) i = n - 1;
  return i;
}

// A compile-time int carried by value (generic lambdas specialise on it).
template <int V>
struct IntC {
  static constexpr int value = V;
};

// Inclusive prefix sum across a 64-lane wavefront, all 64 lanes active.
// Register-to-register DPP moves, no LDS round trip: row_shr 1, 2, 4, 8 scan
// each 16-lane row (a lane whose source lies before its row reads 0), then
// row_bcast:15 adds lane 15's total to row 1 and lane 47's to row 3, and
// row_bcast:31 adds lane 31's total to rows 2 and 3 (the row masks 0xA and
// 0xC leave the other rows at +0).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

// N independent inclusive scans, step by step side by side, so that each DPP
// step's latency is covered by the other scans' steps.
template <int N>
__device__ __forceinline__ void wave_inclusive_scan_n(int (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += __builtin_amdgcn_update_dpp(0, v[i], 0x111, 0xF, 0xF, false);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += __builtin_amdgcn_update_dpp(0, v[i], 0x112, 0xF, 0xF, false);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += __builtin_amdgcn_update_dpp(0, v[i], 0x114, 0xF, 0xF, false);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += __builtin_amdgcn_update_dpp(0, v[i], 0x118, 0xF, 0xF, false);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += __builtin_amdgcn_update_dpp(0, v[i], 0x142, 0xA, 0xF, false);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += __builtin_amdgcn_update_dpp(0, v[i], 0x143, 0xC, 0xF, false);
}

// Lane 63's value, as a wave-uniform scalar (the total of an inclusive scan).
__device__ __forceinline__ int wave_last(int v) { return __builtin_amdgcn_readlane(v, 63); }

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

}  // namespace dwm
