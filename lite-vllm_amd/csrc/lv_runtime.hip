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

extern "C" int lv_device_errors(uint32_t* flags_out, int32_t clear) {
  using namespace lv;
  clear_error();
  if (flags_out) *flags_out = 0;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    set_error("lv_device_errors: hipDeviceSynchronize: %s", hipGetErrorString(e));
    return LV_ERR_HIP;
  }
  int (*const readers[])(uint32_t*, bool) = {read_errors_scatter, read_errors_attention,
                                             read_errors_fused};
  uint32_t all = 0;
  for (auto rd : readers) {
    uint32_t v = 0;
    const int rc = rd(&v, clear != 0);
    if (rc != LV_OK) return rc;
    all |= v;
  }
  if (flags_out) *flags_out = all;
  if (all != 0) {
    set_error("lv_device_errors: kernels met out-of-range indices (clamped):%s%s",
              (all & LV_DEVERR_BLOCK_ID) ? " block-table entry outside [0, num_cache_blocks)"
                                         : "",
              (all & LV_DEVERR_SLOT) ? " slot >= num_blocks * block_size" : "");
    return LV_ERR_DEVICE_INDEX;
  }
  return LV_OK;
}
