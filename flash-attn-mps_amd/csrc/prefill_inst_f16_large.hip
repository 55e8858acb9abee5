// F16T prefill kernel variants, head dims 192/128 and 256 and FP8 K/V.
#include "prefill_kernel.h"

namespace fa_prefill {

PrefillChoice pick_f16_large(int64_t dq, int64_t dv, bool causal, int score, bool win, bool fp8, int mk) {
  return pick_dims_large<F16T>(dq, dv, causal, score, win, fp8, mk);
}

}  // namespace fa_prefill
