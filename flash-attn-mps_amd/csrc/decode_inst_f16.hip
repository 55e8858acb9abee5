// Decode kernel variants with f16 K/V.
#include "decode_kernel.h"

namespace fa_decode {

DecodeKernel pick_decode_f16(int64_t d, int64_t dv, int gt, bool cap, bool alibi, int pk) {
  return pick_dims<F16T, F16T, F16T>(d, dv, gt, cap, alibi, pk);
}

}  // namespace fa_decode
