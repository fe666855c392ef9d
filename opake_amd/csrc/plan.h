// Device-side plan passed from the clip-factor kernel to the clipped-sum
// kernels: the examples with a positive scale, in increasing order.  The GEMM
// walks only these, so examples with scale 0 (clipped to zero, or non-finite
// data) are never read.
//
// Byte layout for a batch of B examples:
//   [0, 4)    int   nactive       number of examples with scale > 0
//   [4, 16)   reserved
//   [16, ..)  int   active[B]     example index of slot j (j < nactive)
#pragma once

#include <stddef.h>

struct ClipPlanView {
  int* nactive;
  int* active;
};

__host__ __device__ inline size_t clip_plan_bytes(int B) {
  size_t b = B > 0 ? (size_t)B : 1;
  return 16 + b * sizeof(int);
}

__host__ __device__ inline ClipPlanView clip_plan_view(void* base, int B) {
  (void)B;
  char* p = (char*)base;
  ClipPlanView v;
  v.nactive = (int*)p;
  v.active = (int*)(p + 16);
  return v;
}
