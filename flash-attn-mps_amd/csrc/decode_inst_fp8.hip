// Decode kernel variants with fp8 K/V.
#include "decode_kernel.h"

namespace fa_decode {

DecodeKernel pick_decode_fp8_bf16(int64_t d, int64_t dv, int gt, bool cap, bool alibi, int pk) {
  return pick_dims<BF16T, E4M3T, E4M3T>(d, dv, gt, cap, alibi, pk);
}

DecodeKernel pick_decode_fp8_f16(int64_t d, int64_t dv, int gt, bool cap, bool alibi, int pk) {
  return pick_dims<F16T, E4M3T, E4M3T>(d, dv, gt, cap, alibi, pk);
}

}  // namespace fa_decode
