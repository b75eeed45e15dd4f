// Host-side plumbing of the C ABI: status strings, per-thread last-error
// text, and the per-device compute-unit count used to size launches.

#include <atomic>
#include <cstdio>
#include <cstring>

#include "rv_device.h"

namespace {

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];  // 0 = not yet queried
thread_local char g_last_error[256] = "";

}  // namespace

namespace rv_host {

int hip_fail(hipError_t err) {
  std::snprintf(g_last_error, sizeof(g_last_error), "%s (%d)",
                hipGetErrorString(err), (int)err);
  return RV_ERR_HIP;
}

int check_launch() {
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? RV_OK : hip_fail(err);
}

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return 256;
  int n = g_cu_count[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
          hipSuccess ||
      n <= 0)
    n = 256;
  g_cu_count[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace rv_host

extern "C" {

const char* rv_status_string(int status) {
  switch (status) {
    case RV_OK: return "ok";
    case RV_ERR_NULL_POINTER: return "null pointer argument";
    case RV_ERR_BAD_SIZE: return "invalid size or sign argument";
    case RV_ERR_UNSUPPORTED: return "unsupported dtype, width or layout";
    case RV_ERR_WORKSPACE: return "workspace missing or too small";
    case RV_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

const char* rv_last_error(void) { return g_last_error; }

int rv_abi_version(void) { return 3; }

}  // extern "C"
