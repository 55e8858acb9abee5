// Device helpers shared by the gfx950 kernels: element codecs, wave
// reductions and the host-side error/launch plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include "../../include/fa_gfx950.h"

#define FA_DEV __device__ __forceinline__

// ------------------------------------------------------------ element types
// Storage tags.  `load` widens one element to fp32, `store` narrows with
// round-to-nearest-even.  E4M3 follows the OCP E4M3FN encoding used by
// torch.float8_e4m3fn: bias 7, no infinities, 0x7F/0xFF are NaN, largest
// finite magnitude 448.

struct F32T  { using storage = float;    static constexpr int bytes = 4; static constexpr int id = FA_F32; };
struct F16T  { using storage = uint16_t; static constexpr int bytes = 2; static constexpr int id = FA_F16; };
struct BF16T { using storage = uint16_t; static constexpr int bytes = 2; static constexpr int id = FA_BF16; };
struct E4M3T { using storage = uint8_t;  static constexpr int bytes = 1; static constexpr int id = FA_E4M3; };

FA_DEV float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

FA_DEV uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

FA_DEV float f16_bits_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

FA_DEV uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// E4M3FN byte -> fp32, exact.
FA_DEV float e4m3_to_f32(uint32_t b) {
  uint32_t e = (b >> 3) & 15u, m = b & 7u;
  uint32_t sign = (b & 0x80u) << 24;
  float x = e == 0 ? (float)m * 0.001953125f : __uint_as_float(((e + 120u) << 23) | (m << 20));
  if (e == 15u && m == 7u) return __uint_as_float(sign | 0x7fc00000u);
  return __uint_as_float(__float_as_uint(x) | sign);
}

// fp32 -> E4M3FN byte: NaN -> sign|0x7F, |a| >= 448 saturates to sign|0x7E,
// otherwise round-to-nearest-even (subnormals in units of 2^-9).
// Integer form: for |a| >= 2^-6 the fp32 magnitude is rounded to 3 mantissa
// bits at bit 20 (ties to even) and its exponent rebiased from 127 to 7, so
// code = (rounded >> 20) - (120 << 3); below 2^-6, fma(|a|, 512, 2^23) rounds
// |a| * 512 to an integer in the low mantissa bits.  Codes past 126 (|a|
// rounding to 480 or more, infinities) clamp to 126.  Host-callable so the
// CPU tests check this very function against the C codec on every fp32 bit
// pattern.
__host__ __device__ __forceinline__ uint32_t e4m3_code(float v) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t mag = bits & 0x7fffffffu;
  const uint32_t normal = (mag + 0x7ffffu + ((mag >> 20) & 1u) - (120u << 23)) >> 20;
  const uint32_t subnormal =
      __builtin_bit_cast(uint32_t, __builtin_fmaf(__builtin_bit_cast(float, mag), 512.0f, 8388608.0f)) - 0x4b000000u;
  uint32_t code = mag < 0x3c800000u ? subnormal : normal;   // 2^-6
  code = code < 126u ? code : 126u;
  code = mag > 0x7f800000u ? 0x7fu : code;                  // NaN
  return sign | code;
}

FA_DEV uint8_t f32_to_e4m3(float v) { return (uint8_t)e4m3_code(v); }

// x / s as the E4M3 encoder needs it, given r = 1/s rounded to nearest (one
// IEEE division per scale): q0 = x r, then one residual step (Markstein)
// q1 = q0 + (x - s q0) r, the residual exact under FMA.  Where |x / s| lies
// in [2^-14, 2^10] q1 is the correctly rounded quotient; elsewhere it is
// within an ulp, which E4M3 cannot see (saturation above 448, zero below
// 2^-11).  q1 is NaN, infinite or zero only where q0 already carries the
// code: x = +-0 (q0 keeps the sign), x = +-inf or overflow (saturates), NaN.
// Valid for scales of magnitude in [2^-100, 2^100] (callers divide directly
// otherwise).  Host-callable: the CPU tests compare it with IEEE division on
// every bf16 and fp16 input over thousands of scales.
__host__ __device__ __forceinline__ float div_by_scale(float x, float s, float r) {
  const float q0 = x * r;
  const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, s, x), r, q0);
  return __builtin_isfinite(q1) && q1 != 0.0f ? q1 : q0;
}

__host__ __device__ __forceinline__ bool scale_in_range(float s) {
  const float a = __builtin_fabsf(s);
  return a >= 0x1p-100f && a <= 0x1p100f;
}

template <typename T> FA_DEV float load_elem(const void* base, int64_t off);
template <> FA_DEV float load_elem<F32T>(const void* base, int64_t off) { return ((const float*)base)[off]; }
template <> FA_DEV float load_elem<F16T>(const void* base, int64_t off) { return f16_bits_to_f32(((const uint16_t*)base)[off]); }
template <> FA_DEV float load_elem<BF16T>(const void* base, int64_t off) { return bf16_bits_to_f32(((const uint16_t*)base)[off]); }
template <> FA_DEV float load_elem<E4M3T>(const void* base, int64_t off) { return e4m3_to_f32(((const uint8_t*)base)[off]); }

template <typename T> FA_DEV void store_elem(void* base, int64_t off, float v);
template <> FA_DEV void store_elem<F32T>(void* base, int64_t off, float v) { ((float*)base)[off] = v; }
template <> FA_DEV void store_elem<F16T>(void* base, int64_t off, float v) { ((uint16_t*)base)[off] = f32_to_f16_bits(v); }
template <> FA_DEV void store_elem<BF16T>(void* base, int64_t off, float v) { ((uint16_t*)base)[off] = f32_to_bf16_bits(v); }

// Runtime-typed element access, for tensors touched once per row.
FA_DEV float load_any(const void* base, int64_t off, int dtype) {
  switch (dtype) {
    case FA_F16: return load_elem<F16T>(base, off);
    case FA_BF16: return load_elem<BF16T>(base, off);
    case FA_E4M3: return load_elem<E4M3T>(base, off);
    default: return load_elem<F32T>(base, off);
  }
}

FA_DEV void store_any(void* base, int64_t off, int dtype, float v) {
  switch (dtype) {
    case FA_F16: store_elem<F16T>(base, off, v); break;
    case FA_BF16: store_elem<BF16T>(base, off, v); break;
    default: store_elem<F32T>(base, off, v); break;
  }
}

// ------------------------------------------------------------ wave helpers
// DPP row controls (GFX9 encoding).
constexpr int DPP_QUAD_XOR1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int DPP_ROW_MIRROR = 0x140;
constexpr int DPP_ROW_HALF_MIRROR = 0x141;

template <int CTRL> FA_DEV float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum / max over each 16-lane row; every lane of the row receives the result.
FA_DEV float row16_sum(float x) {
  x += dpp_mov<DPP_QUAD_XOR1>(x);
  x += dpp_mov<DPP_QUAD_XOR2>(x);
  x += dpp_mov<DPP_ROW_HALF_MIRROR>(x);
  x += dpp_mov<DPP_ROW_MIRROR>(x);
  return x;
}

FA_DEV float row16_max(float x) {
  x = fmaxf(x, dpp_mov<DPP_QUAD_XOR1>(x));
  x = fmaxf(x, dpp_mov<DPP_QUAD_XOR2>(x));
  x = fmaxf(x, dpp_mov<DPP_ROW_HALF_MIRROR>(x));
  x = fmaxf(x, dpp_mov<DPP_ROW_MIRROR>(x));
  return x;
}

FA_DEV int lane_id() {
  return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

FA_DEV float shfl_xor_f(float x, int mask) {
  int lane = lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute(((lane ^ mask) << 2), __float_as_int(x)));
}

FA_DEV float wave_sum(float x) {
  x = row16_sum(x);
  x += shfl_xor_f(x, 16);
  x += shfl_xor_f(x, 32);
  return x;
}

FA_DEV float wave_max(float x) {
  x = row16_max(x);
  x = fmaxf(x, shfl_xor_f(x, 16));
  x = fmaxf(x, shfl_xor_f(x, 32));
  return x;
}

FA_DEV int wave_min_i(int x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = min(x, __shfl_xor(x, m));
  return x;
}
FA_DEV int wave_max_i(int x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = max(x, __shfl_xor(x, m));
  return x;
}
FA_DEV float readlane_f(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Wave-uniform read of memory that no kernel writes while it runs (block
// tables, sequence metadata).  Reading through the constant address space
// lets the compiler use a scalar load, which is tracked separately from the
// vector-memory counter and so never forces a wait on in-flight K/V loads.
FA_DEV int32_t load_invariant_i32(const int32_t* p, int64_t idx) {
  typedef const __attribute__((address_space(4))) int32_t cint32;
  return ((cint32*)p)[idx];
}

FA_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
FA_DEV float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

// ------------------------------------------------------------ host helpers
void fa_set_error(const char* fmt, ...);

#define FA_REQUIRE(cond, ...)             \
  do {                                    \
    if (!(cond)) {                        \
      fa_set_error(__VA_ARGS__);          \
      return FA_ERR_INVALID;              \
    }                                     \
  } while (0)

int fa_check_launch(const char* what);

static inline int64_t fa_ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
