// Host-side error state of the C ABI: one message buffer per calling thread.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.hpp"

namespace {
thread_local char g_last_error[512] = "";
}

namespace sophia {

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error(SOPHIA_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(err));
  g_last_error[0] = '\0';
  return SOPHIA_OK;
}

}  // namespace sophia

extern "C" const char *sophia_last_error(void) { return g_last_error; }

extern "C" int sophia_abi_version(void) { return 107; }
