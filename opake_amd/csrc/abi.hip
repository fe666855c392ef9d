// Library-level entry points of the C ABI.
#include "common.h"

namespace {
thread_local hipError_t g_last_error = hipSuccess;
}

void dpc_record_error(hipError_t e) { g_last_error = e; }

extern "C" int dpc_version(void) { return 207; }

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

// Timing events without the system-scope fence (hipEventDisableSystemFence):
// recording one performs no cache writeback or invalidation, so it neither
// costs the work around it nor inflates the interval it measures.  For
// timing only.
extern "C" int dpc_timing_event_create(void** event) {
  if (!event) return DPC_EINVAL;
  hipEvent_t e = nullptr;
  DPC_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
  *event = (void*)e;
  return DPC_OK;
}

extern "C" int dpc_timing_event_record(void* event, void* stream) {
  if (!event) return DPC_EINVAL;
  DPC_HIP_CHECK(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
  return DPC_OK;
}

extern "C" int dpc_timing_event_elapsed_ms(void* start, void* end, float* ms) {
  if (!start || !end || !ms) return DPC_EINVAL;
  DPC_HIP_CHECK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
  return DPC_OK;
}

extern "C" int dpc_timing_event_destroy(void* event) {
  if (!event) return DPC_OK;
  DPC_HIP_CHECK(hipEventDestroy((hipEvent_t)event));
  return DPC_OK;
}
