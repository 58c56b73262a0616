// Library-wide host helpers: error strings, version, and the MFMA layout self-test.
#include <stdarg.h>

#include "common.h"

namespace fi {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return FI_ERR_HIP;
  }
  return FI_OK;
}

// One wave: c = mfma16x16x32(a, b, 0) with the lane-major fragments of the header.
__global__ __launch_bounds__(64) void selftest_mfma_kernel(const half8* a, const half8* b,
                                                           floatx4* c) {
  const int lane = threadIdx.x;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = mfma16x16x32(a[lane], b[lane], acc);
  c[lane] = acc;
}

}  // namespace fi

extern "C" int fi_version(void) { return 100; }

extern "C" const char* fi_last_error(void) { return fi::g_error; }

extern "C" int fi_selftest_mfma_f16(const void* a, const void* b, void* c, void* stream) {
  fi::clear_error();
  if (!a || !b || !c) {
    fi::set_error("fi_selftest_mfma_f16: null pointer");
    return FI_ERR_INVALID;
  }
  hipLaunchKernelGGL(fi::selftest_mfma_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const fi::half8*)a, (const fi::half8*)b, (fi::floatx4*)c);
  return fi::check_launch("fi_selftest_mfma_f16");
}
