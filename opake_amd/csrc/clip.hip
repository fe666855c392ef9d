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

// Several clip-factor passes in one launch: workgroup k runs group g0 + k's
// pass (its own C and count threshold; outputs at the group's offsets).
constexpr int kClipMaxGroups = 64;
struct ClipGroupArgs {
  double C[kClipMaxGroups];
  float count_threshold[kClipMaxGroups];
};

__global__ void __launch_bounds__(kClipThreads)
clip_factors_groups_kernel(const double* __restrict__ sqnorm, const double* __restrict__ sqerr,
                           int B, int g0, const ClipJob job, const ClipGroupArgs grp) {
  __shared__ int shm[clip_block_lds_ints(kClipThreads / 64)];
  const int k = blockIdx.x, g = g0 + k;
  const size_t gb = (size_t)g * B, gsb = (size_t)g * job.n_guards * B;
  ClipJob j = job;
  j.C = grp.C[k];
  j.count_threshold = grp.count_threshold[k];
  if (j.scale) j.scale += gsb;
  if (j.scale64) j.scale64 += gsb;
  if (j.norms_out) j.norms_out += gb;
  if (j.nclipped) j.nclipped += g;
  if (j.plans) j.plans = (char*)j.plans + (size_t)g * job.n_guards * clip_plan_bytes(B);
  if (j.nonfinite) j.nonfinite += g;
  clip_factors_block(sqnorm + gb, sqerr ? sqerr + gb : nullptr, B, j, shm);
}

}  // namespace

extern "C" size_t dpc_clip_plan_bytes(int B) { return clip_plan_bytes(B); }

extern "C" int dpc_clip_factors_groups(const double* sqnorm, const double* sqerr, int n_groups,
                                       int B, const double* C, int kind, double gamma,
                                       const double* guard_rel, const double* guard_abs,
                                       const int* guard_mult, int n_guards,
                                       const float* count_threshold, float* scale,
                                       double* scale64, float* norms_out, int* nclipped,
                                       void* plan, int* nonfinite, void* stream) {
  if (n_groups < 0 || B < 0) return DPC_EINVAL;
  if (n_groups == 0) return DPC_OK;
  if (!C || !count_threshold || (B > 0 && !sqnorm)) return DPC_EINVAL;
  ClipJob job;
  const int r = clip_job_from_args(C[0], kind, gamma, guard_rel, guard_abs, guard_mult, n_guards,
                                   count_threshold[0], scale, scale64, norms_out, nclipped, plan,
                                   nonfinite, &job);
  if (r != DPC_OK) return r;
  for (int g0 = 0; g0 < n_groups; g0 += kClipMaxGroups) {
    const int n = n_groups - g0 < kClipMaxGroups ? n_groups - g0 : kClipMaxGroups;
    ClipGroupArgs grp = {};
    for (int k = 0; k < n; ++k) {
      grp.C[k] = C[g0 + k];
      grp.count_threshold[k] = count_threshold[g0 + k];
    }
    hipLaunchKernelGGL(clip_factors_groups_kernel, dim3(n), dim3(kClipThreads), 0,
                       (hipStream_t)stream, sqnorm, sqerr, B, g0, job, grp);
    DPC_HIP_CHECK(hipGetLastError());
  }
  return DPC_OK;
}

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
