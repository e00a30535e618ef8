// Error reporting shared by the C entry points.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace fs_host {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return FS_ERR_LAUNCH;
  }
  return FS_OK;
}

}  // namespace fs_host

extern "C" const char* fs_last_error(void) { return fs_host::g_err; }
extern "C" int fs_abi_version(void) { return 12; }

extern "C" size_t fs_sizeof_args(int which) {
  switch (which) {
    case 0: return sizeof(fs_pool_args);
    case 1: return sizeof(fs_corr_args);
    case 2: return sizeof(fs_stats_args);
    case 3: return sizeof(fs_select_args);
    case 4: return sizeof(fs_attn_args);
    case 5: return sizeof(fs_scores_args);
    case 6: return sizeof(fs_rope_pool_args);
    case 7: return sizeof(fs_xattn_args);
    case 8: return sizeof(fs_flex_args);
    default: return 0;
  }
}
