// Library-wide entry points and error state of libvrm_paged.so.
#include <stdarg.h>
#include <stdio.h>

#include "vrm_common.h"

namespace vrm {
namespace {
thread_local char g_last_error[1024] = {0};
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = 0; }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  clear_error();
  return VRM_OK;
}

}  // namespace vrm

extern "C" int vrm_abi_version(void) { return VRM_ABI_VERSION; }

extern "C" const char* vrm_last_error(void) { return vrm::g_last_error; }
