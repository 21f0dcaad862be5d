// Error plumbing and version query of libmlr_attn.so.
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

}  // namespace mlr

extern "C" const char *mlr_last_error(void) {
  return mlr::g_last_error.c_str();
}

extern "C" int mlr_version(void) { return 100; }  // 0.1.0
