// Library-wide host helpers: error strings, version, the CU count per device, and the MFMA
// layout self-test.
#include <stdarg.h>

#include <atomic>

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

// Compute units of the device that runs `stream` (the current device for the null stream),
// queried once per device and cached.
int device_cu_count(hipStream_t stream) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = -1;
  if (stream != nullptr) {
    hipDevice_t d;
    if (hipStreamGetDevice(stream, &d) == hipSuccess) dev = (int)d;
  }
  if (dev < 0 && hipGetDevice(&dev) != hipSuccess) dev = -1;
  if (dev >= 0 && dev < kMaxDevices) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int cus = 0;
  if (dev < 0 || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return 256;  // MI355X
  if (dev < kMaxDevices) cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
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
