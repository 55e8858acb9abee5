// Decode kernel variants with bf16 K/V.
#include "decode_kernel.h"

namespace fa_decode {

DecodeKernel pick_decode_bf16(int64_t d, int64_t dv, int gt, bool cap, bool alibi, int pk) {
  return pick_dims<BF16T, BF16T, BF16T>(d, dv, gt, cap, alibi, pk);
}

}  // namespace fa_decode
