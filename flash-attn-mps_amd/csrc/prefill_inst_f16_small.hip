// F16T prefill kernel variants, 16-bit K/V with head dims up to 128.
#include "prefill_kernel.h"

namespace fa_prefill {

PrefillChoice pick_f16_small(int64_t dq, int64_t dv, bool causal, int score, bool win, int mk) {
  return pick_dims_small<F16T>(dq, dv, causal, score, win, mk);
}

}  // namespace fa_prefill
