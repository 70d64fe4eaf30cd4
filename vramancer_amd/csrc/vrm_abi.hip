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

extern "C" size_t vrm_kv_slab_bytes(int kv_dtype, int KH, int PS, int D) {
  if (KH <= 0 || PS <= 0 || D <= 0 || D > 256) return 0;
  long long row;
  switch (kv_dtype) {
    case VRM_KV_F32: row = 4LL * D; break;
    case VRM_KV_F16:
    case VRM_KV_BF16: row = 2LL * D; break;
    case VRM_KV_I8:
    case VRM_KV_FP8E4M3: row = D; break;
    case VRM_KV_I8_INLINE:
    case VRM_KV_FP8E4M3_INLINE:
      if (PS % 4 || D % 16) return 0;  // the tiled V of the quantized pools
      row = D;
      break;
    default: return 0;
  }
  return (size_t)vrm::pool_geom(kv_dtype, KH, PS, D, row, 1, 1).slab;
}
