// Exhaustive check of the library's f32 -> bf16 conversion (common.h:
// f32_to_bf16_bits / f32x2_to_bf16x2_bits, one v_cvt_pk_bf16_f32 on gfx950)
// against round to nearest even with the quiet-NaN rule, written out in
// integer arithmetic below: every one of the 2^32 f32 bit patterns, in both
// halves of the packed result (the pair (u, ~u) covers each pattern once in
// either half).  Prints the mismatch count and up to 8 examples; the exit
// status is 0 when there are none, 1 on a mismatch, 2 on a HIP error.
// Built beside the library (make -C dw-tpu_amd/csrc); a GPU test runs it.
#include "common.h"

namespace {

// Round to nearest even: adding 0x7FFF plus the kept part's lowest bit
// carries into bit 16 exactly when the dropped 16 bits exceed half, or equal
// half with an odd kept part (a carry out of the mantissa bumps the exponent,
// up to infinity).  A NaN keeps its sign and top payload bits and is made
// quiet (bit 6 of the bf16 pattern, the top mantissa bit).
__device__ uint32_t rne_rule(uint32_t u) {
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

constexpr int kSamples = 8;

__global__ __launch_bounds__(256) void check_kernel(unsigned long long *count, uint32_t *samples) {
  const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;  // 2^24 threads, 256 patterns each
  for (uint32_t j = 0; j < 256; ++j) {
    const uint32_t a = (uint32_t)((t << 8) | j), b = ~a;
    const uint32_t got = dwm::f32x2_to_bf16x2_bits(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    const uint32_t want = rne_rule(a) | (rne_rule(b) << 16);
    if (got != want) {
      const unsigned long long k = atomicAdd(count, 1ull);
      if (k < kSamples) {
        samples[3 * k] = a;
        samples[3 * k + 1] = got;
        samples[3 * k + 2] = want;
      }
    }
  }
}

}  // namespace

int main() {
  unsigned long long *d_count = nullptr;
  uint32_t *d_samples = nullptr;
  if (hipMalloc(&d_count, sizeof(unsigned long long)) != hipSuccess ||
      hipMalloc(&d_samples, 3 * kSamples * sizeof(uint32_t)) != hipSuccess ||
      hipMemset(d_count, 0, sizeof(unsigned long long)) != hipSuccess) {
    fprintf(stderr, "bf16_check: HIP allocation failed\n");
    return 2;
  }
  hipLaunchKernelGGL(check_kernel, dim3(1u << 16), dim3(256), 0, 0, d_count, d_samples);
  unsigned long long count = 0;
  uint32_t samples[3 * kSamples] = {};
  if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(&count, d_count, sizeof(count), hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(samples, d_samples, sizeof(samples), hipMemcpyDeviceToHost) != hipSuccess) {
    fprintf(stderr, "bf16_check: kernel or copy failed\n");
    return 2;
  }
  printf("f32 -> bf16 conversion vs round-to-nearest-even rule over 2^32 patterns x 2 halves: mismatches: %llu\n",
         count);
  for (unsigned long long k = 0; k < count && k < (unsigned long long)kSamples; ++k)
    printf("  input %08x: packed result %08x, rule %08x\n", samples[3 * k], samples[3 * k + 1], samples[3 * k + 2]);
  (void)hipFree(d_count);
  (void)hipFree(d_samples);
  return count == 0 ? 0 : 1;
}
