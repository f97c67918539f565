// Error reporting shared by every extern "C" entry point of libvkwr_amd.
#include <string.h>

#include "vk_capi.h"

namespace vk {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return VKWR_ERR_LAUNCH;
  }
  return VKWR_OK;
}

// Compute units of the current device (cached per device; 256 if the query fails).
int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

}  // namespace vk

extern "C" const char* vkwr_status_string(int status) {
  switch (status) {
    case VKWR_OK: return "ok";
    case VKWR_ERR_INVALID: return "invalid argument";
    case VKWR_ERR_LAUNCH: return "launch failure";
    default: return "unknown status";
  }
}

extern "C" const char* vkwr_last_error(void) { return vk::g_err; }
