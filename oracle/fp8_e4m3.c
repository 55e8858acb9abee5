/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle for the E4M3FN byte codec.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may load it.
 *
 * Restates, in portable C, the codec of SuperMarioYL/flash-attn-mps:
 *   encode: flash_attn_mps/kernels/cache.metal:8-18
 *           NaN -> sign|0x7F; |a| >= 448 -> sign|0x7E; |a| < 2^-6 -> rint(a*512);
 *           otherwise exponent floor(log2 a), mantissa rint(a * 2^(3-e)) - 8 with
 *           round-half-even, code min(((e+7)<<3)+m, 126)
 *   decode: flash_attn_mps/kernels/attention.metal:4-10 and
 *           flash_attn_mps/kernels/attention_decode.metal:10-16
 *           bias 7, subnormal m * 2^-9, 0x7F/0xFF NaN, no infinities.
 * The exponent is read from the IEEE-754 bit pattern rather than computed with
 * log2(), so it is exact for every input.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

uint8_t oracle_e4m3_encode(float v) {
  uint32_t sign = (f32_bits(v) >> 24) & 0x80u;
  float a = fabsf(v);
  if (isnan(a)) return (uint8_t)(sign | 0x7fu);
  if (a >= 448.0f) return (uint8_t)(sign | 0x7eu);
  if (a < 0.015625f) return (uint8_t)(sign | (uint32_t)rintf(a * 512.0f));
  int e = (int)((f32_bits(a) >> 23) & 0xffu) - 127;
  int mant = (int)rintf(ldexpf(a, 3 - e));
  int code = ((e + 7) << 3) + mant - 8;
  if (code > 126) code = 126;
  return (uint8_t)(sign | (uint32_t)code);
}

float oracle_e4m3_decode(uint8_t b) {
  uint32_t e = (b >> 3) & 15u, m = b & 7u;
  float x;
  if (e == 15u && m == 7u) x = NAN;
  else if (e == 0u) x = (float)m * 0.001953125f;
  else x = ldexpf(1.0f + (float)m * 0.125f, (int)e - 7);
  return (b & 0x80u) ? -x : x;
}

/* Vector forms: x / scale[h] quantised per element, like the store kernel. */
void oracle_e4m3_encode_array(const float* x, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_e4m3_encode(x[i]);
}

void oracle_e4m3_encode_scaled(const float* x, const float* scale, int64_t rows, int64_t heads,
                               int64_t dim, int64_t scale_stride, uint8_t* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t h = 0; h < heads; ++h) {
      const float s = scale[h * scale_stride];
      for (int64_t d = 0; d < dim; ++d) {
        const int64_t i = (r * heads + h) * dim + d;
        out[i] = oracle_e4m3_encode(x[i] / s);
      }
    }
}

void oracle_e4m3_decode_array(const uint8_t* b, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_e4m3_decode(b[i]);
}

/* Count encode disagreements with a reference table over every float whose
 * bit pattern is k * stride (k = 0 .. 2^32/stride - 1); used to sweep the
 * whole float line against torch's cast in strided passes. */
int64_t oracle_e4m3_sweep(uint32_t start, uint32_t stride, int64_t count, uint8_t* out) {
  for (int64_t k = 0; k < count; ++k) {
    uint32_t u = start + (uint32_t)k * stride;
    float f;
    memcpy(&f, &u, 4);
    out[k] = oracle_e4m3_encode(f);
  }
  return count;
}
