// Library-level entry points of the C ABI.
#include "common.h"

namespace {
thread_local hipError_t g_last_error = hipSuccess;
}

void dpc_record_error(hipError_t e) { g_last_error = e; }

extern "C" int dpc_version(void) { return 100; }

extern "C" const char* dpc_last_error(void) { return hipGetErrorString(g_last_error); }
