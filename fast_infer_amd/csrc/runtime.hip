// Library-wide host helpers: error strings, version, the CU count per device, the XCD-group
// check and per-stream slots of the kernels that share partial results within an XCD, and the
// MFMA layout self-test.
#include <stdarg.h>

#include <atomic>
#include <mutex>

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

// ---------------------------------------------------------------------------------------
// XCD groups.  The dispatcher deals consecutive workgroups of a launch to the XCDs in turn, so
// workgroups whose block ids are congruent modulo 8 run on one XCD and share its L2: kernels
// that pass partial sums between such workgroups (through stores, an L2 atomic counter and
// L1-bypassing loads) use this only after one probe launch per device has shown it to hold.

constexpr int kMaxDevices = 64;
constexpr int kProbeBlocks = 2048;
__device__ unsigned g_xcd_probe[kProbeBlocks];

__global__ __launch_bounds__(64) void xcd_probe_kernel(unsigned* out) {
  if (threadIdx.x == 0) {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    out[blockIdx.x] = x & 0xf;
  }
}

struct XcdDevice {
  int state = 0;  // 0: not probed, 1: groups share an XCD, -1: they do not (or no answer)
  hipStream_t streams[kXcdPurposes][kXcdMaxSlots] = {};
  int used[kXcdPurposes] = {};
};

static std::mutex& xcd_mutex() {
  static std::mutex mu;
  return mu;
}

static XcdDevice& xcd_device(int dev) {
  static XcdDevice devs[kMaxDevices];
  return devs[dev];
}

static int stream_device(hipStream_t st) {
  hipDevice_t d;
  if (hipStreamGetDevice(st, &d) != hipSuccess) return -1;
  return (int)d < kMaxDevices ? (int)d : -1;
}

// One probe launch on `st`: every block records its XCC_ID into g_xcd_probe (no allocation),
// read back with a synchronous copy.  Called with the device of `st` current.
static bool xcd_probe(hipStream_t st) {
  void* d = nullptr;
  if (hipGetSymbolAddress(&d, HIP_SYMBOL(g_xcd_probe)) != hipSuccess || !d) return false;
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  static unsigned h[kProbeBlocks];
  hipLaunchKernelGGL(xcd_probe_kernel, dim3(kProbeBlocks), dim3(64), 0, st, (unsigned*)d);
  bool ok = hipGetLastError() == hipSuccess &&
            hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, st) == hipSuccess &&
            hipStreamSynchronize(st) == hipSuccess;
  for (int i = 8; ok && i < kProbeBlocks; ++i) ok = h[i] == h[i & 7];
  (void)hipThreadExchangeStreamCaptureMode(&mode);
  return ok;
}

bool xcd_groups_ok(hipStream_t st) {
  const int dev = stream_device(st);
  if (dev < 0) return false;
  std::lock_guard<std::mutex> lock(xcd_mutex());
  XcdDevice& xd = xcd_device(dev);
  if (xd.state == 0) {
    // the probe synchronizes: not while `st` is being captured or an error is pending
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone ||
        hipPeekAtLastError() != hipSuccess)
      return false;
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return false;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return false;
    xd.state = xcd_probe(st) ? 1 : -1;
    if (cur != dev) (void)hipSetDevice(cur);
  }
  return xd.state == 1;
}

int xcd_stream_slot(hipStream_t st, int purpose, int slots) {
  const int dev = stream_device(st);
  if (dev < 0 || purpose < 0 || purpose >= kXcdPurposes || slots > kXcdMaxSlots) return -1;
  std::lock_guard<std::mutex> lock(xcd_mutex());
  XcdDevice& xd = xcd_device(dev);
  for (int i = 0; i < xd.used[purpose]; ++i)
    if (xd.streams[purpose][i] == st) return i;
  if (xd.used[purpose] >= slots) return -1;
  xd.streams[purpose][xd.used[purpose]] = st;
  return xd.used[purpose]++;
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
