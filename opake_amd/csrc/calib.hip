// Measurement helper: the bf16 MFMA throughput the chip sustains on random
// operands.  The published dense peak (2.5 PFLOP/s) holds for operands that
// barely toggle; with random bf16 data the matrix cores draw more power and
// the clock settles lower, so a kernel's fraction of the published peak
// understates how close it is to what the hardware delivers.  This kernel
// runs nothing but 32x32x16 bf16 MFMAs: 8 independent accumulators per wave,
// 8 waves per workgroup (2 per SIMD), operands read once from a caller-filled
// buffer and rotated through 4 registers each.
#include "common.h"

namespace {

constexpr int kCalibThreads = 512;

__global__ void __launch_bounds__(kCalibThreads)
mfma_calib_kernel(const u32x4_t* __restrict__ operands, int iters, float* __restrict__ out) {
  const size_t t = (size_t)blockIdx.x * kCalibThreads + threadIdx.x;
  bf16x8_t a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = __builtin_bit_cast(bf16x8_t, operands[t * 8 + i]);
    b[i] = __builtin_bit_cast(bf16x8_t, operands[t * 8 + 4 + i]);
  }
  f32x16_t acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x16_t{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i & 3], b[(i + (i >> 2)) & 3], acc[i],
                                                       0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += acc[i][threadIdx.x & 15];
  out[t] = s;
}

}  // namespace

extern "C" int dpc_calib_mfma_bf16(const void* operands, int grid, int iters, float* out,
                                   void* stream) {
  if (grid <= 0 || iters <= 0 || !operands || !out) return DPC_EINVAL;
  hipLaunchKernelGGL(mfma_calib_kernel, dim3(grid), dim3(kCalibThreads), 0, (hipStream_t)stream,
                     (const u32x4_t*)operands, iters, out);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}
