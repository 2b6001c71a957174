// Host-side runtime pieces shared by every entry point: the thread-local
// error string behind lv_last_error() and launch checking.
#include <string.h>

#include "lv_common.h"

namespace lv {

static thread_local char g_last_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return LV_ERR_HIP;
  }
  return LV_OK;
}

}  // namespace lv

extern "C" const char* lv_last_error(void) { return lv::g_last_error; }

extern "C" int lv_abi_version(void) { return LV_ABI_VERSION; }
