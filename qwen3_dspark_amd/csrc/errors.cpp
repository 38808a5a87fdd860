// Thread-local error string behind dspark_last_error().
#include <hip/hip_runtime.h>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "common.h"

namespace {
thread_local std::string g_error;
}

namespace dspark {

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}

void clear_error() { g_error.clear(); }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return HIP_FAILURE;
  }
  return OK;
}

}  // namespace dspark

extern "C" const char* dspark_last_error(void) { return g_error.c_str(); }

extern "C" int dspark_abi_version(void) { return 7; }
