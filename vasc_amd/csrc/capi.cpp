// Error plumbing and ABI metadata of libvasc_hip.so.
#include "common.h"

#include <cstring>

namespace vasc {

static thread_local char g_error[512] = "";

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(err));
    return VASC_ERR_HIP;
  }
  return VASC_OK;
}

}  // namespace vasc

extern "C" const char *vasc_last_error(void) { return vasc::g_error; }

extern "C" int vasc_abi_version(void) { return 5; }
