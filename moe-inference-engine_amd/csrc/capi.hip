// Error state and version entry points of libmie_paged.so.
#include <stdarg.h>
#include <stdio.h>

#include "mie_common.h"

namespace mie {

namespace {
thread_local char g_last_error[512] = "";
}

int32_t fail(int32_t code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int32_t check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MIE_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MIE_OK;
}

}  // namespace mie

extern "C" int32_t mie_abi_version(void) { return MIE_ABI_VERSION; }

extern "C" const char* mie_last_error(void) { return mie::g_last_error; }

namespace {
__global__ __launch_bounds__(256) void empty_kernel() {}
}  // namespace

// Measurement only: `workgroups` workgroups of 256 threads of an empty
// kernel, so a caller can time the launch floor that latency-bound calls
// cannot go under.
extern "C" int32_t mie_empty_launch(int32_t workgroups, void* stream) {
  if (workgroups < 1 || workgroups > (1 << 20)) return mie::fail(MIE_ERR_INVALID, "mie_empty_launch: workgroups %d", workgroups);
  mie::clear_error();
  hipLaunchKernelGGL(empty_kernel, dim3(workgroups), dim3(256), 0, static_cast<hipStream_t>(stream));
  return mie::check_launch("mie_empty_launch");
}
