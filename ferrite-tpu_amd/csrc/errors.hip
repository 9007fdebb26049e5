// Per-thread error reporting of the C ABI (ferrite_hip_last_error).
#include <atomic>
#include <string>

#include "common.h"
#include "device_select.h"

namespace ferrite {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FERRITE_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  g_last_error.clear();
  return FERRITE_OK;
}

int stream_device(hipStream_t s) {
  return device_of_stream(
      s, [](const void* st, int* d) { return (int)hipStreamGetDevice(static_cast<hipStream_t>(const_cast<void*>(st)), d); },
      [](int* d) { return (int)hipGetDevice(d); });
}

// Compute units of device `dev` (the current device when dev < 0), looked up
// once per device. Racing first calls store the same value.
int cu_count_of(int dev) {
  static std::atomic<int> cache[64];
  if (dev < 0 && hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int cu_count(hipStream_t s) { return cu_count_of(stream_device(s)); }

DeviceGuard::DeviceGuard(int dev) : prev_(-1) {
  if (dev >= 0 && hipGetDevice(&prev_) == hipSuccess && prev_ != dev && hipSetDevice(dev) == hipSuccess) return;
  prev_ = -1;
}
DeviceGuard::~DeviceGuard() {
  if (prev_ >= 0) (void)hipSetDevice(prev_);
}

int allow_lds(const void* kernel, int bytes, hipStream_t s, const char* what) {
  static OncePerDevice once;
  const int dev = stream_device(s);
  if (dev < 0) return fail(FERRITE_ERR_LAUNCH, std::string(what) + ": cannot tell the stream's device");
  const int rc = once.run(kernel, dev, [&] {
    DeviceGuard on(dev);
    return (int)hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  });
  if (rc != (int)hipSuccess)
    return fail(FERRITE_ERR_LAUNCH, std::string(what) + ": raising the LDS limit to " + std::to_string(bytes) +
                                        " bytes failed: " + hipGetErrorString(static_cast<hipError_t>(rc)));
  return FERRITE_OK;
}

}  // namespace ferrite

extern "C" const char* ferrite_hip_last_error(void) { return ferrite::g_last_error.c_str(); }

extern "C" const char* ferrite_hip_version(void) { return "ferrite_hip 0.1.0 gfx950"; }
