// CPU checks of the product's FP8 store arithmetic (csrc/fa_device.h, the
// functions the store kernels run):
//   e4m3_check enc [stride]  e4m3_code against the oracle's C codec
//                            (oracle/fp8_e4m3.c) on fp32 bit patterns 0, stride, ...
//   e4m3_check div [scales]  div_by_scale against IEEE division x / s on every
//                            finite bf16 and fp16 x for `scales` scales (powers of
//                            two, decimal steps, near-all-ones significands,
//                            pseudo-random): equal E4M3 codes always, equal fp32
//                            bits where |x / s| lies in [2^-14, 2^10]
// Prints the first mismatch and exits 1; exits 0 when everything agrees.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "../../flash-attn-mps_amd/csrc/fa_device.h"

extern "C" uint8_t oracle_e4m3_encode(float v);

static float from_bits(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}

static uint32_t to_bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

static float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
  if (e == 31) return from_bits(sign | 0x7f800000u | (m << 13));
  if (e == 0) return from_bits(sign | to_bits((float)m * 0x1p-24f));
  return from_bits(sign | ((e + 112) << 23) | (m << 13));
}

static float nth_scale(long i) {
  if (i < 64) return from_bits((uint32_t)(95 + i) << 23);                          // 2^-32 .. 2^31
  if (i < 1064) return (float)(i - 63) * 0.001f;                                   // 0.001 .. 1.0
  if (i < 3064) return from_bits(((uint32_t)(100 + i % 56) << 23) | (0x7fffffu - (uint32_t)(i / 56)));
  uint64_t z = (uint64_t)i * 0x9E3779B97F4A7C15ull;                                 // pseudo-random
  z ^= z >> 29;
  return from_bits(0x3c000000u + (uint32_t)(z % (0x44000000u - 0x3c000000u)));
}

static int check_division(long scales) {
  for (long i = 0; i < scales; ++i) {
    const float s = nth_scale(i), r = 1.0f / s;
    for (uint32_t h = 0; h < 65536; ++h) {
      const float xs[2] = {from_bits(h << 16), half_to_float((uint16_t)h)};
      for (float x : xs) {
        if (x != x) continue;
        // The E4M3 codes always agree; inside [2^-14, 2^10] the fp32 quotients too.
        const float want = x / s, got = div_by_scale(x, s, r);
        const float mag = want < 0 ? -want : want;
        const bool exact_window = mag >= 0x1p-14f && mag <= 0x1p10f;
        if (e4m3_code(want) != e4m3_code(got) || (exact_window && to_bits(want) != to_bits(got))) {
          printf("division mismatch: x=%a s=%a: %a vs IEEE %a\n", x, s, got, want);
          return 1;
        }
      }
    }
  }
  printf("division agrees on %ld scales\n", scales);
  return 0;
}

int main(int argc, char** argv) {
  if (argc > 1 && strcmp(argv[1], "div") == 0) return check_division(argc > 2 ? atol(argv[2]) : 4000);
  const uint64_t stride = argc > 2 ? strtoull(argv[2], nullptr, 0) : 1;
  const unsigned nthreads = std::thread::hardware_concurrency() ? std::thread::hardware_concurrency() : 4;
  std::vector<std::thread> pool;
  std::vector<uint64_t> bad(nthreads, ~0ull);
  for (unsigned t = 0; t < nthreads; ++t) {
    pool.emplace_back([&, t] {
      for (uint64_t u = t * stride; u < (1ull << 32); u += nthreads * stride) {
        float f;
        const uint32_t bits = (uint32_t)u;
        memcpy(&f, &bits, 4);
        if ((uint8_t)e4m3_code(f) != oracle_e4m3_encode(f)) {
          bad[t] = u;
          return;
        }
      }
    });
  }
  for (auto& th : pool) th.join();
  for (unsigned t = 0; t < nthreads; ++t)
    if (bad[t] != ~0ull) {
      float f;
      const uint32_t bits = (uint32_t)bad[t];
      memcpy(&f, &bits, 4);
      printf("mismatch at 0x%08x (%g): product 0x%02x oracle 0x%02x\n", bits, f, e4m3_code(f) & 0xff,
             oracle_e4m3_encode(f));
      return 1;
    }
  printf("all %llu patterns agree\n", (unsigned long long)((1ull << 32) / stride));
  return 0;
}
