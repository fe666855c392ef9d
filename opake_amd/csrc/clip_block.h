// Clip factors from per-example squared norms, in float64, plus the active
// example plans consumed by the clipped-sum GEMM -- the workgroup routine
// shared by clip_factors_kernel (clip.hip) and the tail of the split Gram
// kernel (gram.hip).
//
// The scale is the reference's guarded ratio (packages/opake-engine/src/opake/
// api/engine/clipping/_pytree.py:111-157, _streaming.py:84-108), taken from
// an upper bound of the norm when the squared norm comes with an error bound
// (ghost norms: sqnorm + sqerr >= ||g||^2):
//   up = sqrt(max(sq + err, 0));  norm = sqrt(max(sq, 0))
//   ratio = max(C,0)/up  or  max(R,0)/(up + gamma)               (AUTO-S)
//   s = ratio * rel - abs;  s = min(1, s) (fixed only; NaN stays NaN)
//   s = isfinite(s) ? max(s, 0) : 0;  stored as float32, or as the value of
//   the guard's multiply dtype (scale.to(multiply_dtype): for bfloat16 and
//   float16 through float32, as torch converts a float64); `scale64` (when
//   given) keeps s itself for float64 guards.
// `norm` (the estimate) is what the statistics report and count.  Every step
// is one IEEE operation in the order written (contraction off), so the result
// matches a host float64 evaluation bit for bit.
#pragma once

#include "common.h"
#include "plan.h"

constexpr int kClipMaxGuards = 4;

struct ClipGuards {
  double rel[kClipMaxGuards];
  double abs_[kClipMaxGuards];
  int mult[kClipMaxGuards];  // the multiply dtype the scale is converted to
};

// What a clip-factor pass computes and where it writes: everything but the
// squared norms.  Any output pointer may be null.
struct ClipJob {
  double C;
  int kind;
  double gamma;
  ClipGuards guards;
  int n_guards;
  float count_threshold;
  float* scale;      // [n_guards, B]
  double* scale64;   // [n_guards, B]
  float* norms_out;  // [B]
  int* nclipped;     // [1]
  void* plans;       // n_guards plans of clip_plan_bytes(B)
  int* nonfinite;    // [1]: examples whose squared norm (or bound) is not
                     // finite, stored with system scope (may be pinned host
                     // memory the host reads once the pass has completed)
};

// s.to(multiply dtype) as a float: torch converts a float64 to bfloat16 or
// float16 through float32 (each step to nearest even).
DPC_DEVICE float clip_scale_in(double s, int mult) {
  const float f = (float)s;
  if (mult == DPC_BF16) return round_to_bf16(f);
  if (mult == DPC_F16) return round_to_f16(f);
  return f;
}

#pragma clang fp contract(off)
DPC_DEVICE double clip_guarded_scale(double sq, double err, double C, int kind, double gamma,
                                     double rel, double abs_, double* norm_out) {
  const double est = sq < 0.0 ? 0.0 : sq;  // NaN stays NaN
  *norm_out = sqrt(est);
  double up = sq + err;
  up = up < 0.0 ? 0.0 : up;
  const double norm = sqrt(up);
  double bound = C > 0.0 ? C : 0.0;
  double ratio = (kind == DPC_SCALE_AUTO_S) ? bound / (norm + gamma) : bound / norm;
  double s = ratio * rel;
  s = s - abs_;
  if (kind != DPC_SCALE_AUTO_S) s = (s > 1.0) ? 1.0 : s;  // torch.minimum keeps NaN
  if (!isfinite(s)) s = 0.0;
  return s < 0.0 ? 0.0 : s;
}
#pragma clang fp contract(on)

// LDS words clip_factors_block needs for a workgroup of `nw` waves.
DPC_HOST_DEVICE int clip_block_lds_ints(int nw) { return 3 * nw + 2; }

// The clip-factor pass over B examples by one whole workgroup (every thread
// calls it; it synchronises the workgroup).  sq / err (err nullable) may be
// global or LDS arrays.  `shm`: clip_block_lds_ints(waves) ints of LDS.
//
// Guard g's pass computes its scales and lists its active examples in plan g
// (see plan.h): the fast ones from the front of `active` in increasing order,
// the others from its back, in increasing order read backwards.  Each list is
// an ordered compaction: a ballot within a wave, wave offsets through LDS.
// The norms and the clipped count come from guard 0's pass.
__device__ inline void clip_factors_block(const double* sq, const double* err, int B,
                                          const ClipJob& job, int* shm) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nw = blockDim.x >> 6;
  int* wave_counts = shm;
  int* clipped_counts = shm + nw;
  int* slow_counts = shm + 2 * nw;
  int* base = shm + 3 * nw;
  int* base_slow = base + 1;
  int clipped_local = 0, nonfinite_local = 0;
  for (int i = tid; i < B; i += blockDim.x)
    nonfinite_local += !(isfinite(sq[i]) && (err == nullptr || isfinite(err[i])));
  const bool fast_ok = (double)B * job.C <= (double)DPC_FAST_BC_MAX;
  for (int g = 0; g < job.n_guards; ++g) {
    const bool have_plan = job.plans != nullptr;
    ClipPlanView plan = clip_plan_view((char*)job.plans + (size_t)g * clip_plan_bytes(B), B);
    if (tid == 0) {
      *base = 0;
      *base_slow = 0;
    }
    for (int start = 0; start < B; start += blockDim.x) {
      const int i = start + tid;
      bool fast = false, slow = false;
      if (i < B) {
        double norm;
        const double s = clip_guarded_scale(sq[i], err ? err[i] : 0.0, job.C, job.kind,
                                            job.gamma, job.guards.rel[g], job.guards.abs_[g],
                                            &norm);
        const float sf = clip_scale_in(s, job.guards.mult[g]);
        if (job.scale) job.scale[(size_t)g * B + i] = sf;
        if (job.scale64)
          job.scale64[(size_t)g * B + i] = job.guards.mult[g] == DPC_F64 ? s : (double)sf;
        if (g == 0) {
          if (job.norms_out) job.norms_out[i] = (float)norm;
          if ((float)norm > job.count_threshold) ++clipped_local;
        }
        fast = sf > 0.0f && fast_ok && sf >= DPC_FAST_SCALE_MIN && sf <= DPC_FAST_SCALE_MAX;
        slow = sf > 0.0f && !fast;
      }
      const unsigned long long mf = __ballot(fast), ms = __ballot(slow);
      const unsigned long long below = (1ull << lane) - 1ull;
      if (lane == 0) {
        wave_counts[w] = __popcll(mf);
        slow_counts[w] = __popcll(ms);
      }
      __syncthreads();
      int of = *base, os = *base_slow;
      for (int v = 0; v < w; ++v) {
        of += wave_counts[v];
        os += slow_counts[v];
      }
      if (have_plan && fast) plan.active[of + __popcll(mf & below)] = i;
      if (have_plan && slow) plan.active[B - 1 - (os + __popcll(ms & below))] = i;
      __syncthreads();
      if (tid == 0) {
        for (int v = 0; v < nw; ++v) {
          *base += wave_counts[v];
          *base_slow += slow_counts[v];
        }
      }
      __syncthreads();
    }
    if (tid == 0 && have_plan) {
      *plan.nactive = *base + *base_slow;
      *plan.nfast = *base;
    }
    __syncthreads();
  }
  for (int off = 32; off > 0; off >>= 1) {
    clipped_local += __shfl_down(clipped_local, off, 64);
    nonfinite_local += __shfl_down(nonfinite_local, off, 64);
  }
  if (lane == 0) {
    clipped_counts[w] = clipped_local;
    wave_counts[w] = nonfinite_local;
  }
  __syncthreads();
  if (tid == 0) {
    int total = 0, bad = 0;
    for (int v = 0; v < nw; ++v) {
      total += clipped_counts[v];
      bad += wave_counts[v];
    }
    if (job.nclipped) *job.nclipped = total;
    if (job.nonfinite)
      __hip_atomic_store(job.nonfinite, bad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// Host side: the job of a dpc_clip_factors-style call; DPC_OK or DPC_EINVAL.
inline int clip_job_from_args(double C, int kind, double gamma, const double* guard_rel,
                              const double* guard_abs, const int* guard_mult, int n_guards,
                              float count_threshold, float* scale, double* scale64,
                              float* norms_out, int* nclipped, void* plan, int* nonfinite,
                              ClipJob* job) {
  if (n_guards < 1 || n_guards > kClipMaxGuards || !guard_rel || !guard_abs) return DPC_EINVAL;
  if (kind != DPC_SCALE_FIXED && kind != DPC_SCALE_AUTO_S) return DPC_EINVAL;
  if (plan && !scale) return DPC_EINVAL;
  ClipJob j = {};
  j.C = C;
  j.kind = kind;
  j.gamma = gamma;
  j.n_guards = n_guards;
  j.count_threshold = count_threshold;
  for (int g = 0; g < n_guards; ++g) {
    j.guards.rel[g] = guard_rel[g];
    j.guards.abs_[g] = guard_abs[g];
    j.guards.mult[g] = guard_mult ? guard_mult[g] : DPC_F32;
    if (!known_dtype(j.guards.mult[g])) return DPC_EINVAL;
  }
  j.scale = scale;
  j.scale64 = scale64;
  j.norms_out = norms_out;
  j.nclipped = nclipped;
  j.plans = plan;
  j.nonfinite = nonfinite;
  *job = j;
  return DPC_OK;
}
