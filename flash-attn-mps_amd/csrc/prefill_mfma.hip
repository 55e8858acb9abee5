// MFMA prefill entry points.  The gfx950 MFMA kernel is added in the next
// change; until then every combination reports "not supported" and the
// dispatcher runs the generic kernel.
#include "attn_common.h"

extern "C" int fa_prefill_supported(const fa_attn_args* a) {
  (void)a;
  return 0;
}

extern "C" int fa_prefill_fwd(const fa_attn_args* a, void* stream) {
  (void)stream;
  int rc = fa_validate_attn(a, "fa_prefill_fwd");
  if (rc) return rc;
  fa_set_error("fa_prefill_fwd: combination not supported by the MFMA kernel");
  return FA_ERR_UNSUPPORTED;
}
