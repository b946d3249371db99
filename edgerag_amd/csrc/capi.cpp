// Thread-local error state and version string for the C ABI.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace edgerag {

namespace {
thread_local char g_error[1024] = "";
}

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(EDGERAG_EHIP, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
  }
  return EDGERAG_OK;
}

}  // namespace edgerag

extern "C" const char* edgerag_last_error(void) { return edgerag::g_error; }

extern "C" const char* edgerag_version(void) { return "edgerag_amd 0.1.0 gfx950"; }
