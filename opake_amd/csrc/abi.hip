// Library-level entry points of the C ABI.
#include "common.h"

namespace {
thread_local hipError_t g_last_error = hipSuccess;
}

void dpc_record_error(hipError_t e) { g_last_error = e; }

extern "C" int dpc_version(void) { return 203; }

extern "C" const char* dpc_last_error(void) { return hipGetErrorString(g_last_error); }

namespace {
// Words of a small table travel as kernel arguments (<= 4 KiB per launch).
constexpr int kWordsPerLaunch = 960;
struct TableWords {
  uint32_t w[kWordsPerLaunch];
};

__global__ void __launch_bounds__(256) write_words_kernel(uint32_t* __restrict__ dst,
                                                          TableWords words, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = words.w[i];
}
}  // namespace

extern "C" int dpc_write_words(void* dst, const uint32_t* host_words, int n, void* stream) {
  if (n < 0 || (n > 0 && (!dst || !host_words))) return DPC_EINVAL;
  for (int base = 0; base < n; base += kWordsPerLaunch) {
    const int m = n - base < kWordsPerLaunch ? n - base : kWordsPerLaunch;
    TableWords words;
    for (int i = 0; i < m; ++i) words.w[i] = host_words[base + i];
    hipLaunchKernelGGL(write_words_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream,
                       (uint32_t*)dst + base, words, m);
    DPC_HIP_CHECK(hipGetLastError());
  }
  return DPC_OK;
}
