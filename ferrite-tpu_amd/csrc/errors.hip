// Per-thread error reporting of the C ABI (ferrite_hip_last_error).
#include <atomic>
#include <string>

#include "common.h"

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

// Compute units of the current device, looked up once per device. Racing
// first calls store the same value.
int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace ferrite

extern "C" const char* ferrite_hip_last_error(void) { return ferrite::g_last_error.c_str(); }

extern "C" const char* ferrite_hip_version(void) { return "ferrite_hip 0.1.0 gfx950"; }
