// Library-wide C ABI plumbing: version, thread-local error text, device count.
#include <string>

#include "wc_common.h"

namespace wc {

static thread_local std::string g_last_error;

int32_t set_error(int32_t code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error.assign(buf);
  return code;
}

void clear_error() { g_last_error.clear(); }

int32_t check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(static_cast<int32_t>(e), "%s: launch failed: %s", what, hipGetErrorString(e));
  return WC_OK;
}

}  // namespace wc

extern "C" {

int32_t wc_abi_version(void) { return WC_ABI_VERSION; }

const char* wc_last_error(void) { return wc::g_last_error.c_str(); }

int32_t wc_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

}  // extern "C"
