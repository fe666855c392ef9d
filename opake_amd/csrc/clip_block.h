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

// What the plans and counts need to know of one example, as flag bits: for
// guard g, bit 2 g (fast: the GEMM's pipelined path may carry the scale) and
// bit 2 g + 1 (slow: a positive scale it cannot); the norm above the count
// threshold; a non-finite squared norm or bound.
constexpr int kClipFlagClipped = 1 << 8;
constexpr int kClipFlagNonfinite = 1 << 9;

// One example's clip factors under every guard (the scale s and its value in
// the multiply dtype sf), its norm estimate and its flag bits, before they
// are stored.  `err` is ignored without `has_err`.
struct ClipExample {
  int flags;
  float norm;
  float sf[kClipMaxGuards];
  double s[kClipMaxGuards];
};

DPC_DEVICE ClipExample clip_example_eval(double sq, double err, bool has_err, int B,
                                         const ClipJob& job) {
  ClipExample e;
  e.flags = (isfinite(sq) && (!has_err || isfinite(err))) ? 0 : kClipFlagNonfinite;
  e.norm = 0.0f;
  const bool fast_ok = (double)B * job.C <= (double)DPC_FAST_BC_MAX;
#pragma unroll
  for (int g = 0; g < kClipMaxGuards; ++g) {
    e.s[g] = 0.0;
    e.sf[g] = 0.0f;
    if (g >= job.n_guards) continue;
    double norm;
    const double s = clip_guarded_scale(sq, has_err ? err : 0.0, job.C, job.kind, job.gamma,
                                        job.guards.rel[g], job.guards.abs_[g], &norm);
    const float sf = clip_scale_in(s, job.guards.mult[g]);
    e.s[g] = s;
    e.sf[g] = sf;
    if (g == 0) {
      e.norm = (float)norm;
      if ((float)norm > job.count_threshold) e.flags |= kClipFlagClipped;
    }
    const bool fast =
        sf > 0.0f && fast_ok && sf >= DPC_FAST_SCALE_MIN && sf <= DPC_FAST_SCALE_MAX;
    const bool slow = sf > 0.0f && !fast;
    e.flags |= (fast ? 1 : 0) << (2 * g);
    e.flags |= (slow ? 2 : 0) << (2 * g);
  }
  return e;
}

// Stores example i's factors to the job's scale / scale64 / norms_out.
DPC_DEVICE void clip_example_store(const ClipExample& e, int i, int B, const ClipJob& job) {
#pragma unroll
  for (int g = 0; g < kClipMaxGuards; ++g) {
    if (g >= job.n_guards) continue;
    if (job.scale) job.scale[(size_t)g * B + i] = e.sf[g];
    if (job.scale64)
      job.scale64[(size_t)g * B + i] = job.guards.mult[g] == DPC_F64 ? e.s[g] : (double)e.sf[g];
  }
  if (job.norms_out) job.norms_out[i] = e.norm;
}

// Both: stores example i's factors and returns its flag bits.
DPC_DEVICE int clip_example(double sq, double err, bool has_err, int i, int B,
                            const ClipJob& job) {
  const ClipExample e = clip_example_eval(sq, err, has_err, B, job);
  clip_example_store(e, i, B, job);
  return e.flags;
}

// The running state of one wave's plan compaction: the size of each guard's
// fast (2 g) and slow (2 g + 1) list so far, and the counts.
struct ClipLists {
  int size[2 * kClipMaxGuards];
  int clipped;
  int nonfinite;
};

// One wave (all 64 lanes, uniform control): places examples i0 .. i0 + n - 1,
// whose flag bits are flags[0 .. n - 1], in every guard's plan after the
// examples placed so far, 64 at a time.  Guard g's plan lists its active
// examples (see plan.h): the fast ones from the front of `active` in
// increasing order, the others from its back, in increasing order read
// backwards -- an ordered compaction by ballots, the list sizes uniform.
// The clipped count is guard 0's.
DPC_DEVICE void clip_compact_wave(const int* flags, int n, int i0, int B, const ClipJob& job,
                                  ClipLists& st) {
  const int lane = threadIdx.x & 63;
  const unsigned long long below = (1ull << lane) - 1ull;
  const int nl = 2 * job.n_guards;
  for (int c = 0; c < n; c += 64) {
    const int f = c + lane < n ? flags[c + lane] : 0;
    st.clipped += __popcll(__ballot((f & kClipFlagClipped) != 0));
    st.nonfinite += __popcll(__ballot((f & kClipFlagNonfinite) != 0));
#pragma unroll
    for (int l = 0; l < 2 * kClipMaxGuards; ++l) {
      if (l >= nl) break;
      const unsigned long long m = __ballot((f >> l) & 1);
      if (job.plans && ((f >> l) & 1)) {
        const int o = st.size[l] + __popcll(m & below);
        ClipPlanView plan =
            clip_plan_view((char*)job.plans + (size_t)(l / 2) * clip_plan_bytes(B), B);
        plan.active[(l & 1) ? B - 1 - o : o] = i0 + c + lane;
      }
      st.size[l] += __popcll(m);
    }
  }
}

// One wave, after the last clip_compact_wave: the list lengths and counts.
DPC_DEVICE void clip_finish_wave(const ClipLists& st, int B, const ClipJob& job) {
  const int lane = threadIdx.x & 63;
  if (job.plans && lane < job.n_guards) {
    int fast = 0, slow = 0;
#pragma unroll
    for (int g = 0; g < kClipMaxGuards; ++g) {
      fast = lane == g ? st.size[2 * g] : fast;
      slow = lane == g ? st.size[2 * g + 1] : slow;
    }
    ClipPlanView plan = clip_plan_view((char*)job.plans + (size_t)lane * clip_plan_bytes(B), B);
    *plan.nactive = fast + slow;
    *plan.nfast = fast;
  }
  if (lane == 0) {
    if (job.nclipped) *job.nclipped = st.clipped;
    if (job.nonfinite)
      __hip_atomic_store(job.nonfinite, st.nonfinite, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// LDS words clip_factors_block needs for a workgroup of `nw` waves.
DPC_HOST_DEVICE constexpr int clip_block_lds_ints(int nw) { return 64 * nw; }

// The whole clip-factor pass over B examples by one workgroup (every thread
// calls it; it synchronises the workgroup): the factors of a round of
// blockDim examples in parallel (clip_example), their flags through LDS,
// then wave 0 places them in the plans.  The barriers order LDS only, so the
// output stores are never waited for.  sq / err (err nullable) may be global
// or LDS arrays.  `shm`: clip_block_lds_ints(waves) ints of LDS.
__device__ inline void clip_factors_block(const double* sq, const double* err, int B,
                                          const ClipJob& job, int* shm) {
  const int tid = threadIdx.x;
  ClipLists st = {};
  for (int start = 0; start < B; start += (int)blockDim.x) {
    const int i = start + tid;
    if (i < B) shm[tid] = clip_example(sq[i], err ? err[i] : 0.0, err != nullptr, i, B, job);
    dpc_lds_barrier();
    if (tid < 64) clip_compact_wave(shm, min((int)blockDim.x, B - start), start, B, job, st);
    dpc_lds_barrier();
  }
  if (tid < 64) clip_finish_wave(st, B, job);
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
