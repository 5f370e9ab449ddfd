// Library-wide entry points of the threadcut HIP library: error reporting,
// ABI version, and the cached device query used by the split heuristic.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "tc_common.hpp"

namespace tc {

namespace {
thread_local char g_last_error[512] = {0};

constexpr int kMaxDevices = 64;
std::mutex g_cu_mutex;
int g_cus[kMaxDevices] = {0};
}  // namespace

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return TC_OK;
  return fail(TC_ERR_HIP, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}

int current_device_cus(int* cus_out) {
  int dev = 0;
  int rc = hip_status(hipGetDevice(&dev), "hipGetDevice");
  if (rc != TC_OK) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(TC_ERR_HIP, "device id %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_cu_mutex);
  if (g_cus[dev] == 0) {
    int cus = 0;
    rc = hip_status(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
                    "hipDeviceGetAttribute(MultiprocessorCount)");
    if (rc != TC_OK) return rc;
    g_cus[dev] = cus > 0 ? cus : 1;
  }
  *cus_out = g_cus[dev];
  return TC_OK;
}

}  // namespace tc

extern "C" {

const char* tc_strerror(int code) {
  switch (code) {
    case TC_OK: return "success";
    case TC_ERR_INVALID_ARGUMENT: return "invalid argument";
    case TC_ERR_UNSUPPORTED: return "unsupported shape or dtype";
    case TC_ERR_ALIGNMENT: return "pointer or stride not 16-byte aligned";
    case TC_ERR_WORKSPACE: return "workspace too small";
    case TC_ERR_HIP: return "HIP runtime error";
    default: return "unknown error";
  }
}

const char* tc_last_error(void) { return tc::g_last_error; }

int tc_abi_version(void) { return 2; }

}  // extern "C"
