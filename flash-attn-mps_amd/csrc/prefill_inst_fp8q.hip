// Prefill kernel variants with E4M3 queries over E4M3 K/V (S on the FP8
// MFMA), fp16 or bf16 output, head dims 64, 128 and 256.
#include "prefill_kernel.h"

namespace fa_prefill {

PrefillChoice pick_fp8q(int out_dtype, int64_t dq, int64_t dv, bool causal, int score, bool win) {
  if (out_dtype == FA_F16) return pick_dims_fp8q<F16T>(dq, dv, causal, score, win);
  if (out_dtype == FA_BF16) return pick_dims_fp8q<BF16T>(dq, dv, causal, score, win);
  return PrefillChoice{nullptr, 0, 0, 0};
}

}  // namespace fa_prefill
