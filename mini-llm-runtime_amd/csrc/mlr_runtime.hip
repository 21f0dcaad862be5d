// Error plumbing and version query of libmlr_attn.so.
#include <atomic>
#include <string>

#include "mlr_common.h"

namespace mlr {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(MLR_ERR_HIP, "%s: kernel launch failed: %s", what,
                     hipGetErrorString(err));
  }
  return MLR_OK;
}

int current_device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cus_of[kMaxDevices];  // 0: not queried yet
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = cus_of[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    // Threads that race here store the same value.
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    cus_of[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace mlr

extern "C" const char *mlr_last_error(void) {
  return mlr::g_last_error.c_str();
}

extern "C" int mlr_version(void) { return 100; }  // 0.1.0
