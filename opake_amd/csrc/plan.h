// Device-side plan passed from the clip-factor kernel to the clipped-sum
// kernels: the examples with a positive scale.  The GEMM walks only these, so
// examples with scale 0 (clipped to zero, or non-finite data) are never read.
// active[0 .. nfast - 1] holds, in increasing order, the examples whose scale
// the bf16 GEMM may apply to its fp32 accumulators (2^-64 <= scale <= 2^32,
// and B * C <= 2^55, which bound the unscaled partial sums and the rescale
// ratios); active[B - 1], active[B - 2], ... down to
// active[B - (nactive - nfast)] the others (gradient norms beyond ~1.8e19 C,
// or AUTO-S scales above 2^32), in increasing order, whose G rows the GEMM
// multiplies by the power of two of their scale (exact) before the product,
// the scale's mantissa going to the accumulators.  dpc_clip_factors writes
// one plan per guard, consecutively, clip_plan_bytes(B) bytes each.
//
// Byte layout for a batch of B examples:
//   [0, 4)    int   nactive       number of examples with scale > 0
//   [4, 8)    int   nfast         number of them in the front list
//   [8, 16)   reserved
//   [16, ..)  int   active[B]
#pragma once

#include <stddef.h>

struct ClipPlanView {
  int* nactive;
  int* nfast;
  int* active;
};

// Smallest and largest scale the GEMM applies to its accumulators, and the
// largest B * C for which it does (see above).
#define DPC_FAST_SCALE_MIN 5.421010862427522e-20f /* 2^-64 */
#define DPC_FAST_SCALE_MAX 4294967296.0f /* 2^32 */
#define DPC_FAST_BC_MAX 3.602879701896397e16 /* 2^55 */

__host__ __device__ inline size_t clip_plan_bytes(int B) {
  size_t b = B > 0 ? (size_t)B : 1;
  return 16 + b * sizeof(int);
}

__host__ __device__ inline ClipPlanView clip_plan_view(void* base, int B) {
  (void)B;
  char* p = (char*)base;
  ClipPlanView v;
  v.nactive = (int*)p;
  v.nfast = (int*)(p + 4);
  v.active = (int*)(p + 16);
  return v;
}
