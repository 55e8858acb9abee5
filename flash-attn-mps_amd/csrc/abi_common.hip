// ABI bookkeeping shared by every entry point: version, struct sizes and the
// per-thread error message returned by fa_last_error().
#include <stdarg.h>
#include <stdio.h>

#include "fa_device.h"

static thread_local char g_fa_error[1024] = "";

void fa_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_fa_error, sizeof(g_fa_error), fmt, ap);
  va_end(ap);
}

int fa_check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    fa_set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return FA_ERR_LAUNCH;
  }
  return FA_OK;
}

extern "C" int fa_abi_version(void) { return FA_ABI_VERSION; }

extern "C" void fa_struct_sizes(int64_t* sizes6) {
  sizes6[0] = (int64_t)sizeof(fa_store_args);
  sizes6[1] = (int64_t)sizeof(fa_append_args);
  sizes6[2] = (int64_t)sizeof(fa_rotary_args);
  sizes6[3] = (int64_t)sizeof(fa_attn_args);
  sizes6[4] = (int64_t)sizeof(fa_merge_pair_args);
  sizes6[5] = (int64_t)sizeof(fa_merge_partials_args);
}

extern "C" const char* fa_last_error(void) { return g_fa_error; }
