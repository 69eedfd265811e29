// ABI bookkeeping: version and the thread-local last error.
#include <stdio.h>
#include <string.h>

#include "abi_internal.hpp"

namespace vaayu {

static thread_local char g_err[512];

int set_error(int code, const char* msg) {
  snprintf(g_err, sizeof g_err, "%s", msg);
  return code;
}

void clear_error() { g_err[0] = 0; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return 0;
  snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e));
  return (int)e;
}

}  // namespace vaayu

extern "C" int vaayu_abi_version(void) { return VAAYU_ABI_VERSION; }

extern "C" const char* vaayu_last_error(void) { return vaayu::g_err; }
