// MFMA issue-rate probe: how many bf16 MFMAs a SIMD completes per cycle with
// one, two or three waves issuing them, alone or with fp4 -> bf16 converts
// (v_cvt_scalef32_pk_bf16_fp4, the gmm's weight decode) between them.
// 256 blocks of 4 x W waves (one block per CU, W waves per SIMD); every wave
// runs ITERS rounds of 16 MFMAs on independent accumulator chains (8 chains
// of 16x16x32, or 4 of 32x32x16) and C converts per round on 16 independent
// registers, all in registers (no memory traffic in the loop).  Prints, per
// case, the aggregate PFLOP/s from HIP events, the shader cycles (s_memtime)
// per MFMA on one SIMD, and the shader clock over the launch (the chip is
// power-limited: a denser MFMA load runs at a lower clock); exits 0, or 2 on
// a HIP error.
// Built beside the library (make -C dw-tpu_amd/csrc).
#include "common.h"

namespace {

using dwm::bf16x8_t;
using dwm::f32x16_t;
using dwm::f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4v;

constexpr int kIters = 2048;
constexpr int kBlocks = 256;

// SHAPE 0: 16x16x32 bf16 (8 chains); 1: 32x32x16 bf16 (4 chains).
template <int SHAPE, int CVT>
__global__ void mfma_kernel(uint32_t *out, uint64_t *cycles, float scale) {
  uint32_t r[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) r[i] = threadIdx.x * 2654435761u + i * 40503u;
  f32x4_t acc4[8];
  f32x16_t acc16[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc4[i] = f32x4_t{0.f, 0.f, 0.f, (float)i};
#pragma unroll
  for (int i = 0; i < 4; ++i) acc16[i] = f32x16_t{};
  const bf16x8_t a = __builtin_bit_cast(bf16x8_t, u32x4v{r[0], r[1], r[2], r[3]});
  const bf16x8_t b = __builtin_bit_cast(bf16x8_t, u32x4v{r[4], r[5], r[6], r[7]});
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < kIters; ++it) {
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      if constexpr (SHAPE == 0) acc4[m % 8] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc4[m % 8], 0, 0, 0);
      else acc16[m % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc16[m % 4], 0, 0, 0);
      // C converts per 16 MFMAs, spread evenly between them.
#pragma unroll
      for (int c = 0; c < CVT / 16; ++c) {
        const int i = (m * (CVT / 16) + c) % 16;
        r[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(r[i], scale, 0));
      }
    }
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) x ^= r[i];
#pragma unroll
  for (int i = 0; i < 8; ++i) x ^= __builtin_bit_cast(uint32_t, acc4[i][0]);
#pragma unroll
  for (int i = 0; i < 4; ++i) x ^= __builtin_bit_cast(uint32_t, acc16[i][0]);
  out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = x;
  if ((threadIdx.x & 63) == 0) cycles[(int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)] = t1 - t0;
}

bool ok(hipError_t e) { return e == hipSuccess; }

template <int SHAPE, int CVT>
bool run(uint32_t *out, uint64_t *cycles, uint64_t *host_cycles, int wps) {
  const int threads = 256 * wps;
  hipEvent_t e0, e1;
  if (!ok(hipEventCreate(&e0)) || !ok(hipEventCreate(&e1))) return false;
  bool good = true;
  for (int i = 0; i < 2 && good; ++i) {  // warm, then timed
    good = ok(hipEventRecord(e0));
    hipLaunchKernelGGL((mfma_kernel<SHAPE, CVT>), dim3(kBlocks), dim3(threads), 0, 0, out, cycles, 1.0f);
    good = good && ok(hipGetLastError()) && ok(hipEventRecord(e1)) && ok(hipEventSynchronize(e1));
  }
  float ms = 0;
  const int waves = kBlocks * 4 * wps;
  good = good && ok(hipEventElapsedTime(&ms, e0, e1)) &&
         ok(hipMemcpy(host_cycles, cycles, waves * sizeof(uint64_t), hipMemcpyDeviceToHost));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (!good) return false;
  double mean_cycles = 0;
  for (int w = 0; w < waves; ++w) mean_cycles += (double)host_cycles[w] / waves;
  const double mfma_per_wave = 16.0 * kIters;
  const double flops = (double)waves * mfma_per_wave * (SHAPE == 0 ? 2.0 * 16 * 16 * 32 : 2.0 * 32 * 32 * 16);
  // The shader clock: the waves' s_memtime spans over the launch's wall time.
  printf("%-9s %2d converts per 16 MFMAs, %d wave%s per SIMD: %5.2f PFLOP/s, %5.1f cycles per MFMA per SIMD, "
         "clock %.2f GHz\n",
         SHAPE == 0 ? "16x16x32" : "32x32x16", CVT, wps, wps > 1 ? "s" : " ", flops / (ms * 1e-3) / 1e15,
         mean_cycles / mfma_per_wave / wps, mean_cycles / (ms * 1e-3) / 1e9);
  fflush(stdout);
  return true;
}

}  // namespace

int main() {
  uint32_t *out = nullptr;
  uint64_t *cycles = nullptr;
  static uint64_t host_cycles[kBlocks * 12];
  if (!ok(hipMalloc(&out, kBlocks * 768 * sizeof(uint32_t))) || !ok(hipMalloc(&cycles, sizeof(host_cycles)))) {
    fprintf(stderr, "mfma_probe: HIP allocation failed\n");
    return 2;
  }
  bool good = true;
  for (int wps = 1; wps <= 3 && good; ++wps) {
    good = good && run<0, 0>(out, cycles, host_cycles, wps);
    good = good && run<0, 16>(out, cycles, host_cycles, wps);
    good = good && run<0, 32>(out, cycles, host_cycles, wps);
    good = good && run<1, 0>(out, cycles, host_cycles, wps);
  }
  (void)hipFree(out);
  (void)hipFree(cycles);
  if (!good) {
    fprintf(stderr, "mfma_probe: HIP error\n");
    return 2;
  }
  return 0;
}
