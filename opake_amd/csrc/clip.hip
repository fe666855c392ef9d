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
  __shared__ int slow_counts[kClipThreads / 64];
  __shared__ int base, base_slow;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nw = blockDim.x >> 6;
  if (tid == 0) base = 0;
  int clipped_local = 0;
  // One pass computes the scales and lists the active examples (see
  // plan.h): the fast ones from the front of `active` in increasing order,
  // the others from its back, in increasing order read backwards.  Each list
  // is an ordered compaction: a ballot within a wave, wave offsets through
  // LDS.
  const bool fast_ok = (double)B * C <= (double)DPC_FAST_BC_MAX;
  if (tid == 0) base_slow = 0;
  for (int start = 0; start < B; start += blockDim.x) {
    const int i = start + tid;
    bool fast = false, slow = false;
    if (i < B) {
      double norm;
      float s0 = 0.0f;
      for (int g = 0; g < n_guards; ++g) {
        double s = guarded_scale(sqnorm[i], C, kind, gamma, guards.rel[g], guards.abs_[g], &norm);
        float sf = (float)s;
        if (scale) scale[(size_t)g * B + i] = sf;
        if (g == 0) s0 = sf;
      }
      if (norms_out) norms_out[i] = (float)norm;
      if ((float)norm > count_threshold) ++clipped_local;
      fast = s0 > 0.0f && fast_ok && s0 >= DPC_FAST_SCALE_MIN;
      slow = s0 > 0.0f && !fast;
    }
    const unsigned long long mf = __ballot(fast), ms = __ballot(slow);
    const unsigned long long below = (1ull << lane) - 1ull;
    if (lane == 0) {
      wave_counts[w] = __popcll(mf);
      slow_counts[w] = __popcll(ms);
    }
    __syncthreads();
    int of = base, os = base_slow;
    for (int v = 0; v < w; ++v) {
      of += wave_counts[v];
      os += slow_counts[v];
    }
    if (have_plan && fast) plan.active[of + __popcll(mf & below)] = i;
    if (have_plan && slow) plan.active[B - 1 - (os + __popcll(ms & below))] = i;
    __syncthreads();
    if (tid == 0) {
      for (int v = 0; v < nw; ++v) {
        base += wave_counts[v];
        base_slow += slow_counts[v];
      }
    }
    __syncthreads();
  }
  for (int off = 32; off > 0; off >>= 1) clipped_local += __shfl_down(clipped_local, off, 64);
  if (lane == 0) clipped_counts[w] = clipped_local;
  __syncthreads();
  if (tid == 0) {
    int total = 0;
    for (int v = 0; v < nw; ++v) total += clipped_counts[v];
    if (nclipped) *nclipped = total;
    if (have_plan) {
      *plan.nactive = base + base_slow;
      *plan.nfast = base;
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
