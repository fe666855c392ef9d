// Clip factors from per-example squared norms, in float64, plus the active
// example plans consumed by the clipped-sum GEMM: one workgroup running
// clip_factors_block (clip_block.h, which states the arithmetic).
#include "clip_block.h"

namespace {

constexpr int kClipThreads = 1024;

__global__ void __launch_bounds__(kClipThreads)
clip_factors_kernel(const double* __restrict__ sqnorm, const double* __restrict__ sqerr, int B,
                    const ClipJob job) {
  __shared__ int shm[clip_block_lds_ints(kClipThreads / 64)];
  clip_factors_block(sqnorm, sqerr, B, job, shm);
}

}  // namespace

extern "C" size_t dpc_clip_plan_bytes(int B) { return clip_plan_bytes(B); }

extern "C" int dpc_clip_factors(const double* sqnorm, const double* sqerr, int B, double C,
                                int kind, double gamma,
                                const double* guard_rel, const double* guard_abs,
                                const int* guard_mult, int n_guards, float count_threshold,
                                float* scale, double* scale64, float* norms_out, int* nclipped,
                                void* plan, int* nonfinite, void* stream) {
  if (B < 0 || (B > 0 && !sqnorm)) return DPC_EINVAL;
  ClipJob job;
  const int r = clip_job_from_args(C, kind, gamma, guard_rel, guard_abs, guard_mult, n_guards,
                                   count_threshold, scale, scale64, norms_out, nclipped, plan,
                                   nonfinite, &job);
  if (r != DPC_OK) return r;
  hipLaunchKernelGGL(clip_factors_kernel, dim3(1), dim3(kClipThreads), 0, (hipStream_t)stream,
                     sqnorm, sqerr, B, job);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}
