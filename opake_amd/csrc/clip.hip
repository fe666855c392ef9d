// Clip factors from per-example squared norms, in float64, plus the active
// example plan consumed by the clipped-sum GEMM.
//
// The scale is the reference's guarded ratio (packages/opake-engine/src/opake/
// api/engine/clipping/_pytree.py:111-157, _streaming.py:84-108):
//   ratio = max(C,0)/norm  or  max(R,0)/(norm + gamma)           (AUTO-S)
//   s = ratio * rel - abs;  s = min(1, s) (fixed only; NaN stays NaN)
//   s = isfinite(s) ? max(s, 0) : 0;  stored as float32.
// Every step is one IEEE operation in the order written (contraction off), so
// the result matches a host float64 evaluation bit for bit.
#include "common.h"
#include "plan.h"

namespace {

constexpr int kClipThreads = 1024;
constexpr int kMaxGuards = 4;

struct Guards {
  double rel[kMaxGuards];
  double abs_[kMaxGuards];
};

#pragma clang fp contract(off)
__device__ double guarded_scale(double sq, double C, int kind, double gamma, double rel,
                                double abs_, double* norm_out) {
  double norm = sqrt(sq);
  *norm_out = norm;
  double bound = C > 0.0 ? C : 0.0;
  double ratio = (kind == DPC_SCALE_AUTO_S) ? bound / (norm + gamma) : bound / norm;
  double s = ratio * rel;
  s = s - abs_;
  if (kind != DPC_SCALE_AUTO_S) s = (s > 1.0) ? 1.0 : s;  // torch.minimum keeps NaN
  if (!isfinite(s)) s = 0.0;
  return s < 0.0 ? 0.0 : s;
}

__global__ void __launch_bounds__(kClipThreads)
clip_factors_kernel(const double* __restrict__ sqnorm, int B, double C, int kind, double gamma,
                    Guards guards, int n_guards, float count_threshold, float* __restrict__ scale,
                    float* __restrict__ norms_out, int* __restrict__ nclipped,
                    void* __restrict__ plan_base) {
  const bool have_plan = plan_base != nullptr;
  ClipPlanView plan = clip_plan_view(plan_base, B);
  __shared__ int wave_counts[kClipThreads / 64];
  __shared__ int clipped_counts[kClipThreads / 64];
  __shared__ int base;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nw = blockDim.x >> 6;
  if (tid == 0) base = 0;
  int clipped_local = 0;
  // Pass 0 computes the scales and lists the fast examples (see plan.h);
  // pass 1 lists the other active ones after them.  Each listing is an
  // ordered compaction: a ballot within a wave, wave offsets through LDS.
  const bool fast_ok = (double)B * C <= (double)DPC_FAST_BC_MAX;
  int nfast = 0;
  for (int pass = 0; pass < (have_plan ? 2 : 1); ++pass) {
    for (int start = 0; start < B; start += blockDim.x) {
      const int i = start + tid;
      bool take = false;
      if (i < B) {
        float s0;
        if (pass == 0) {
          double norm;
          for (int g = 0; g < n_guards; ++g) {
            double s = guarded_scale(sqnorm[i], C, kind, gamma, guards.rel[g], guards.abs_[g], &norm);
            float sf = (float)s;
            if (scale) scale[(size_t)g * B + i] = sf;
            if (g == 0) s0 = sf;
          }
          if (norms_out) norms_out[i] = (float)norm;
          if ((float)norm > count_threshold) ++clipped_local;
        } else {
          s0 = scale[i];
        }
        const bool fast = fast_ok && s0 >= DPC_FAST_SCALE_MIN;
        take = s0 > 0.0f && (pass == 0 ? fast : !fast);
      }
      unsigned long long mask = __ballot(take);
      int before = __popcll(mask & ((1ull << lane) - 1ull));
      if (lane == 0) wave_counts[w] = __popcll(mask);
      __syncthreads();
      int offset = base;
      for (int v = 0; v < w; ++v) offset += wave_counts[v];
      if (have_plan && take) plan.active[offset + before] = i;
      __syncthreads();
      if (tid == 0) {
        int total = 0;
        for (int v = 0; v < nw; ++v) total += wave_counts[v];
        base += total;
      }
      __syncthreads();
    }
    if (pass == 0) nfast = base;  // every thread reads base after the barrier above
  }
  for (int off = 32; off > 0; off >>= 1) clipped_local += __shfl_down(clipped_local, off, 64);
  if (lane == 0) clipped_counts[w] = clipped_local;
  __syncthreads();
  if (tid == 0) {
    int total = 0;
    for (int v = 0; v < nw; ++v) total += clipped_counts[v];
    if (nclipped) *nclipped = total;
    if (have_plan) {
      *plan.nactive = base;
      *plan.nfast = nfast;
    }
  }
}

}  // namespace

extern "C" size_t dpc_clip_plan_bytes(int B) { return clip_plan_bytes(B); }

extern "C" int dpc_clip_factors(const double* sqnorm, int B, double C, int kind, double gamma,
                                const double* guard_rel, const double* guard_abs, int n_guards,
                                float count_threshold, float* scale, float* norms_out,
                                int* nclipped, void* plan, void* stream) {
  if (B < 0 || n_guards < 1 || n_guards > kMaxGuards || !guard_rel || !guard_abs) {
    return DPC_EINVAL;
  }
  if (kind != DPC_SCALE_FIXED && kind != DPC_SCALE_AUTO_S) return DPC_EINVAL;
  if (B > 0 && !sqnorm) return DPC_EINVAL;
  if (plan && !scale) return DPC_EINVAL;
  Guards guards = {};
  for (int g = 0; g < n_guards; ++g) {
    guards.rel[g] = guard_rel[g];
    guards.abs_[g] = guard_abs[g];
  }
  hipLaunchKernelGGL(clip_factors_kernel, dim3(1), dim3(kClipThreads), 0, (hipStream_t)stream,
                     sqnorm, B, C, kind, gamma, guards, n_guards, count_threshold,
                     scale, norms_out, nclipped, plan);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}
