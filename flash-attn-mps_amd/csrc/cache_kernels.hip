// Slot-mapped KV-cache writes, FA2-style appends and rotary embedding.
//
// store_kvcache follows flash_attn_mps/kernels/cache.metal:20-39 (slot ->
// page/offset, skip slot < 0 or >= pages*P, optional E4M3 quantisation of
// x / scale[h]); append follows cache.metal:41-56 and rotary cache.metal:58-76.
// The gfx950 kernels here move 16-byte vectors per lane when the head
// dimension is contiguous and aligned, and fall back to one element per lane
// for arbitrary strides.
#include <type_traits>

#include "fa_device.h"

namespace {

struct StoreDescK {
  const void* x;
  void* cache;
  const float* scale;
  int64_t heads, dim, chunks;   // chunks = dim / VEC
  int64_t xs[3], cs[4];
  int64_t scale_stride;
};

struct StoreParams {
  StoreDescK d[2];
  const void* slots;
  int64_t slot_stride, tokens, page_size, num_slots;
  int32_t ndesc;
};

template <typename IT>
FA_DEV int64_t read_slot(const void* slots, int64_t t, int64_t stride) {
  return (int64_t)((const IT*)slots)[t * stride];
}

// One lane handles VEC consecutive head-dim elements of one (token, head).
// Same-dtype stores copy raw bits (NaN payloads and signed zeros preserved).
template <typename XT, bool FP8, typename IT, int VEC>
__global__ __launch_bounds__(256) void store_kernel(const StoreParams p) {
  const StoreDescK& d = p.d[blockIdx.y];
  const int64_t per_token = d.heads * d.chunks;
  const int64_t total = p.tokens * per_token;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / per_token;
    const int64_t rem = i - t * per_token;
    const int64_t h = rem / d.chunks;
    const int64_t e = (rem - h * d.chunks) * VEC;
    const int64_t slot = read_slot<IT>(p.slots, t, p.slot_stride);
    if (slot < 0 || slot >= p.num_slots) continue;
    int64_t block, offset;
    if (p.num_slots <= 0xffffffffll) {
      const uint32_t s32 = (uint32_t)slot, ps = (uint32_t)p.page_size;
      block = s32 / ps;
      offset = s32 - (uint32_t)block * ps;
    } else {
      block = slot / p.page_size;
      offset = slot - block * p.page_size;
    }
    const int64_t src = t * d.xs[0] + h * d.xs[1] + e * d.xs[2];
    const int64_t dst = block * d.cs[0] + offset * d.cs[1] + h * d.cs[2] + e * d.cs[3];
    if constexpr (!FP8) {
      using S = typename XT::storage;
      if constexpr (VEC * sizeof(S) == 16) {
        *(uint4*)((S*)d.cache + dst) = *(const uint4*)((const S*)d.x + src);
      } else {
        static_assert(VEC == 1, "vector width");
        ((S*)d.cache)[dst] = ((const S*)d.x)[src];
      }
    } else {
      const float scale = d.scale[h * d.scale_stride];
      uint8_t* out = (uint8_t*)d.cache + dst;
      if constexpr (VEC == 1) {
        out[0] = f32_to_e4m3(load_elem<XT>(d.x, src) / scale);
      } else {
        // VEC elements of XT = 16 bytes in, VEC bytes out.
        uint4 raw = *(const uint4*)((const typename XT::storage*)d.x + src);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
        uint8_t q[VEC];
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          float f;
          if constexpr (XT::bytes == 4) f = __uint_as_float(w[j]);
          else {
            const uint32_t half = (w[j / 2] >> (16 * (j & 1))) & 0xffffu;
            f = XT::id == FA_BF16 ? bf16_bits_to_f32(half) : f16_bits_to_f32(half);
          }
          q[j] = f32_to_e4m3(f / scale);
        }
        if constexpr (VEC == 8) {
          uint2 o;
          o.x = q[0] | (q[1] << 8) | (q[2] << 16) | ((uint32_t)q[3] << 24);
          o.y = q[4] | (q[5] << 8) | (q[6] << 16) | ((uint32_t)q[7] << 24);
          *(uint2*)out = o;
        } else {
          *(uint32_t*)out = q[0] | (q[1] << 8) | (q[2] << 16) | ((uint32_t)q[3] << 24);
        }
      }
    }
  }
}

// Vector path by whole token rows.  A wave stores one token at a time: lane l
// owns the (head, 16-byte chunk) tasks l, l + 64, ... (TPL per lane, fixed for
// the kernel, so no element does any division), the slot is read once per
// token and split into page and row with a shift (power-of-two pages) or one
// 32-bit division.  FP8: x / scale[h] (correctly rounded, by div_by_scale
// with the scale's reciprocal) then the hardware E4M3 conversion (the
// integer encoder's byte for every non-NaN input: checked on all 2^32 fp32
// patterns; 2.4x fewer VALU instructions per element, the store 2-3%
// faster), VEC codes stored as one 8- or 4-byte word.
// Streaming (non-temporal) accesses: the token rows are read once and the
// cache rows written once, so neither is kept in the caches (1.5% faster
// than ordinary loads and stores on a 590K-token FP8 store).
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t nt_u32x2 __attribute__((ext_vector_type(2)));

FA_DEV uint4 load16_nt(const void* p) {
  const nt_u32x4 v = __builtin_nontemporal_load((const nt_u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
FA_DEV void store16_nt(void* p, uint4 v) { __builtin_nontemporal_store(nt_u32x4{v.x, v.y, v.z, v.w}, (nt_u32x4*)p); }
FA_DEV void store8_nt(void* p, uint2 v) { __builtin_nontemporal_store(nt_u32x2{v.x, v.y}, (nt_u32x2*)p); }
FA_DEV void store4_nt(void* p, uint32_t v) { __builtin_nontemporal_store(v, (uint32_t*)p); }

template <typename XT, bool FP8, typename IT, int TPL>
__global__ __launch_bounds__(256) void store_rows_kernel(const StoreParams p, const int log2_page) {
  constexpr int VEC = 16 / XT::bytes;
  using S = typename XT::storage;
  const StoreDescK& d = p.d[blockIdx.y];
  const int lane = threadIdx.x & 63;
  const int tasks = (int)(d.heads * d.chunks);
  int64_t src[TPL], dst[TPL];
  float scale[TPL], recip[TPL];
  bool on[TPL], fast_div[TPL];
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    const int task = lane + 64 * i;
    on[i] = task < tasks;
    const int h = on[i] ? task / (int)d.chunks : 0, c = on[i] ? task % (int)d.chunks : 0;
    src[i] = h * d.xs[1] + (int64_t)c * VEC * d.xs[2];
    dst[i] = h * d.cs[2] + (int64_t)c * VEC * d.cs[3];
    scale[i] = FP8 ? d.scale[h * d.scale_stride] : 1.0f;
    recip[i] = 1.0f / scale[i];                 // IEEE: rounded to nearest
    fast_div[i] = scale_in_range(scale[i]);
  }
  // All of this wave's scales in range (the usual case): the loop below is
  // instantiated with the reciprocal division only.
  bool all_fast = true;
#pragma unroll
  for (int i = 0; i < TPL; ++i) all_fast = all_fast && fast_div[i];
  all_fast = __all(all_fast);
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  auto run = [&](auto fast) {
    for (int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < p.tokens; t += nwaves) {
      const int64_t slot = read_slot<IT>(p.slots, t, p.slot_stride);
      if (slot < 0 || slot >= p.num_slots) continue;
      int64_t block, offset;
      if (log2_page >= 0) {
        block = slot >> log2_page;
        offset = slot & ((1ll << log2_page) - 1);
      } else if (p.num_slots <= 0xffffffffll) {
        const uint32_t s32 = (uint32_t)slot, ps = (uint32_t)p.page_size;
        block = s32 / ps;
        offset = s32 - (uint32_t)block * ps;
      } else {
        block = slot / p.page_size;
        offset = slot - block * p.page_size;
      }
      const S* xrow = (const S*)d.x + t * d.xs[0];
      const int64_t crow = block * d.cs[0] + offset * d.cs[1];
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        if (!on[i]) continue;
        const uint4 raw = load16_nt(xrow + src[i]);
        if constexpr (!FP8) {
          store16_nt((S*)d.cache + crow + dst[i], raw);
        } else {
          const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
          uint32_t packed[VEC / 4];
          float qs[VEC];
          bool anynan = false;
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            float f;
            if constexpr (XT::bytes == 4) f = __uint_as_float(w[j]);
            else {
              const uint32_t half = (w[j / 2] >> (16 * (j & 1))) & 0xffffu;
              f = XT::id == FA_BF16 ? bf16_bits_to_f32(half) : f16_bits_to_f32(half);
            }
            float q;
            if constexpr (decltype(fast)::value) q = div_by_scale(f, scale[i], recip[i]);
            else q = f / scale[i];
            qs[j] = q;
            anynan |= q != q;
          }
          // Hardware conversion of |q| clamped to 448 (v_med3, then
          // v_cvt_pk_fp8_f32, round to nearest even): the byte e4m3_code
          // gives for every non-NaN fp32 value; NaN lanes take e4m3_code.
#pragma unroll
          for (int j = 0; j < VEC; j += 4) {
            int v = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(qs[j], -448.0f, 448.0f),
                                                    __builtin_amdgcn_fmed3f(qs[j + 1], -448.0f, 448.0f), 0, false);
            v = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(qs[j + 2], -448.0f, 448.0f),
                                                __builtin_amdgcn_fmed3f(qs[j + 3], -448.0f, 448.0f), v, true);
            packed[j / 4] = (uint32_t)v;
          }
          if (__builtin_expect(anynan, 0)) {
#pragma unroll
            for (int j = 0; j < VEC; ++j)
              if (qs[j] != qs[j]) {
                const uint32_t code = e4m3_code(qs[j]) & 0xffu;
                packed[j / 4] = (packed[j / 4] & ~(0xffu << (8 * (j & 3)))) | (code << (8 * (j & 3)));
              }
          }
          uint8_t* out = (uint8_t*)d.cache + crow + dst[i];
          if constexpr (VEC == 8) store8_nt(out, make_uint2(packed[0], packed[1]));
          else store4_nt(out, packed[0]);
        }
      }
    }
  };
  if (!FP8 || all_fast) run(std::true_type());
  else run(std::false_type());
}

int elem_bytes(int dtype) { return dtype == FA_F32 ? 4 : dtype == FA_E4M3 ? 1 : 2; }

bool aligned(const void* p, int64_t a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }

template <typename XT, bool FP8, typename IT>
int launch_store(const StoreParams& p, bool vec, hipStream_t stream) {
  constexpr int VEC = 16 / XT::bytes;
  if (vec) {
    // Token rows of at most 512 tasks (8 per lane) take the row kernel.
    int64_t tasks = 0;
    for (int i = 0; i < p.ndesc; ++i) tasks = p.d[i].heads * p.d[i].chunks > tasks ? p.d[i].heads * p.d[i].chunks : tasks;
    if (tasks <= 512) {
      int log2_page = -1;
      if ((p.page_size & (p.page_size - 1)) == 0)
        for (log2_page = 0; (1ll << log2_page) < p.page_size; ++log2_page) {}
      int64_t blocks = fa_ceil_div(p.tokens, 4);
      // 64 workgroups per CU at most; each wave then loops over tokens.  (On
      // a 590K-token FP8 store 16K workgroups per descriptor ran 7% faster
      // than 2K, and 64K or one per four tokens were slower again.)
      if (blocks > 16384) blocks = 16384;
      const dim3 grid((unsigned)blocks, (unsigned)p.ndesc);
      const int tpl = (int)fa_ceil_div(tasks, 64);
      if (tpl == 1) hipLaunchKernelGGL((store_rows_kernel<XT, FP8, IT, 1>), grid, dim3(256), 0, stream, p, log2_page);
      else if (tpl == 2) hipLaunchKernelGGL((store_rows_kernel<XT, FP8, IT, 2>), grid, dim3(256), 0, stream, p, log2_page);
      else if (tpl <= 4) hipLaunchKernelGGL((store_rows_kernel<XT, FP8, IT, 4>), grid, dim3(256), 0, stream, p, log2_page);
      else hipLaunchKernelGGL((store_rows_kernel<XT, FP8, IT, 8>), grid, dim3(256), 0, stream, p, log2_page);
      return fa_check_launch("fa_store_kvcache");
    }
  }
  int64_t work = 0;
  for (int i = 0; i < p.ndesc; ++i) {
    const int64_t w = p.tokens * p.d[i].heads * p.d[i].chunks;
    work = w > work ? w : work;
  }
  int64_t blocks = fa_ceil_div(work, 256);
  if (blocks > 65535 * 8) blocks = 65535 * 8;
  if (blocks < 1) blocks = 1;
  dim3 grid((unsigned)blocks, (unsigned)p.ndesc);
  if (vec)
    hipLaunchKernelGGL((store_kernel<XT, FP8, IT, VEC>), grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((store_kernel<XT, FP8, IT, 1>), grid, dim3(256), 0, stream, p);
  return fa_check_launch("fa_store_kvcache");
}

template <typename XT, bool FP8>
int launch_store_idx(const StoreParams& p, int slot_dtype, bool vec, hipStream_t s) {
  return slot_dtype == FA_I64 ? launch_store<XT, FP8, int64_t>(p, vec, s)
                              : launch_store<XT, FP8, int32_t>(p, vec, s);
}

// ------------------------------------------------------------------ append

struct AppendParams {
  StoreDescK d[2];
  int64_t xb[2];                 // batch strides of the two inputs
  const int32_t* lengths;
  const int32_t* batch_index;
  const int32_t* table;
  int64_t batch, new_tokens, page_size, num_blocks, table_rows, table_cols;
  int32_t ndesc;
};

template <typename XT, bool FP8>
__global__ __launch_bounds__(256) void append_kernel(const AppendParams p) {
  const int which = blockIdx.y;
  const StoreDescK& d = p.d[which];
  const int64_t total = p.batch * p.new_tokens * d.heads * d.dim;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = i % d.dim;
    const int64_t h = (i / d.dim) % d.heads;
    const int64_t bj = i / (d.dim * d.heads);
    const int64_t j = bj % p.new_tokens, b = bj / p.new_tokens;
    const bool paged = p.table != nullptr;
    const int64_t row = (!paged && p.batch_index) ? (int64_t)p.batch_index[b] : b;
    const int64_t pos = (int64_t)p.lengths[b] + j;
    const int64_t rows = paged ? p.table_rows : p.num_blocks;
    const int64_t limit = paged ? p.table_cols * p.page_size : p.page_size;
    if (row < 0 || row >= rows || pos < 0 || pos >= limit) continue;
    const int64_t block = paged ? (int64_t)p.table[row * p.table_cols + pos / p.page_size] : row;
    const int64_t offset = paged ? pos % p.page_size : pos;
    if (block < 0 || block >= p.num_blocks) continue;
    const int64_t src = b * p.xb[which] + j * d.xs[0] + h * d.xs[1] + e * d.xs[2];
    const int64_t dst = block * d.cs[0] + offset * d.cs[1] + h * d.cs[2] + e * d.cs[3];
    if constexpr (FP8) {
      ((uint8_t*)d.cache)[dst] = f32_to_e4m3(load_elem<XT>(d.x, src) / d.scale[h * d.scale_stride]);
    } else {
      using S = typename XT::storage;
      ((S*)d.cache)[dst] = ((const S*)d.x)[src];
    }
  }
}

// ------------------------------------------------------------------ rotary

struct RotaryParams {
  const void* x;
  void* out;
  const float* cos_t;
  const float* sin_t;
  const int32_t* lengths;
  int64_t batch, seq, heads, dim, half, rows;
  int64_t xs[4];
  int32_t interleaved, advance;
};

template <typename XT>
__global__ __launch_bounds__(256) void rotary_kernel(const RotaryParams p) {
  const int64_t total = p.batch * p.seq * p.heads * p.dim;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t d = i % p.dim;
    const int64_t h = (i / p.dim) % p.heads;
    const int64_t bj = i / (p.dim * p.heads);
    const int64_t j = bj % p.seq, b = bj / p.seq;
    const int64_t src = b * p.xs[0] + j * p.xs[1] + h * p.xs[2] + d * p.xs[3];
    using S = typename XT::storage;
    if (d >= 2 * p.half) {
      ((S*)p.out)[i] = ((const S*)p.x)[src];
      continue;
    }
    int64_t pair, other;
    bool second;
    if (p.interleaved) {
      pair = d / 2;
      second = (d & 1) != 0;
      other = second ? d - 1 : d + 1;
    } else {
      second = d >= p.half;
      pair = second ? d - p.half : d;
      other = second ? d - p.half : d + p.half;
    }
    const int64_t pos = (int64_t)p.lengths[b] + (p.advance ? j : 0);
    // Lengths live on the device, so the host cannot check them against the
    // table: a position with no cos/sin row rotates to NaN instead of
    // reading past the table.
    if (pos < 0 || pos >= p.rows) {
      store_elem<XT>(p.out, i, __builtin_nanf(""));
      continue;
    }
    const float c = p.cos_t[pos * p.half + pair], s = p.sin_t[pos * p.half + pair];
    const float x = load_elem<XT>(p.x, src);
    const float y = load_elem<XT>(p.x, b * p.xs[0] + j * p.xs[1] + h * p.xs[2] + other * p.xs[3]);
    const float r = second ? x * c + y * s : x * c - y * s;
    store_elem<XT>(p.out, i, r);
  }
}

StoreDescK to_desc(const fa_store_desc& s, int64_t vec) {
  StoreDescK d;
  d.x = s.x;
  d.cache = s.cache;
  d.scale = s.scale;
  d.heads = s.heads;
  d.dim = s.dim;
  d.chunks = s.dim / vec;
  for (int i = 0; i < 3; ++i) d.xs[i] = s.x_stride[i];
  for (int i = 0; i < 4; ++i) d.cs[i] = s.cache_stride[i];
  d.scale_stride = s.scale_stride;
  return d;
}

bool desc_vectorizable(const fa_store_desc& s, int vec_elems) {
  const int xb = elem_bytes(s.x_dtype), cb = elem_bytes(s.cache_dtype);
  if (s.x_stride[2] != 1 || s.cache_stride[3] != 1 || s.dim % vec_elems) return false;
  if (!aligned(s.x, 16) || !aligned(s.cache, vec_elems * cb)) return false;
  for (int i = 0; i < 2; ++i)
    if ((s.x_stride[i] * xb) % 16) return false;
  for (int i = 0; i < 3; ++i)
    if ((s.cache_stride[i] * cb) % (vec_elems * cb)) return false;
  return true;
}

}  // namespace

extern "C" int fa_store_kvcache(const fa_store_args* a, void* stream) {
  FA_REQUIRE(a != nullptr, "fa_store_kvcache: null args");
  FA_REQUIRE(a->slots != nullptr, "fa_store_kvcache: null slot mapping");
  FA_REQUIRE(a->slot_dtype == FA_I32 || a->slot_dtype == FA_I64, "fa_store_kvcache: slots must be int32/int64");
  FA_REQUIRE(a->page_size > 0 && a->num_pages >= 0 && a->tokens >= 0, "fa_store_kvcache: bad sizes");
  const int ndesc = a->kv[1].x ? 2 : 1;
  const int xdt = a->kv[0].x_dtype, cdt = a->kv[0].cache_dtype;
  for (int i = 0; i < ndesc; ++i) {
    const fa_store_desc& s = a->kv[i];
    FA_REQUIRE(s.x && s.cache, "fa_store_kvcache: null tensor %d", i);
    FA_REQUIRE(s.x_dtype == xdt && s.cache_dtype == cdt, "fa_store_kvcache: K and V must share dtypes");
    FA_REQUIRE(s.x_dtype == FA_F16 || s.x_dtype == FA_BF16 || s.x_dtype == FA_F32,
               "fa_store_kvcache: input dtype must be f16/bf16/f32");
    FA_REQUIRE(s.cache_dtype == s.x_dtype || s.cache_dtype == FA_E4M3,
               "fa_store_kvcache: cache dtype must match input or be E4M3");
    FA_REQUIRE(s.cache_dtype != FA_E4M3 || s.scale != nullptr, "fa_store_kvcache: E4M3 cache needs a scale");
    FA_REQUIRE(s.heads > 0 && s.dim > 0, "fa_store_kvcache: empty head/dim");
  }
  if (a->tokens == 0) return FA_OK;
  const bool fp8 = cdt == FA_E4M3;
  const int vec_elems = 16 / elem_bytes(xdt);
  bool vec = true;
  for (int i = 0; i < ndesc; ++i) vec = vec && desc_vectorizable(a->kv[i], vec_elems);
  StoreParams p;
  for (int i = 0; i < 2; ++i) p.d[i] = to_desc(a->kv[i < ndesc ? i : 0], vec ? vec_elems : 1);
  p.slots = a->slots;
  p.slot_stride = a->slot_stride;
  p.tokens = a->tokens;
  p.page_size = a->page_size;
  p.num_slots = a->num_pages * a->page_size;
  p.ndesc = ndesc;
  hipStream_t s = (hipStream_t)stream;
  switch (xdt) {
    case FA_F16: return fp8 ? launch_store_idx<F16T, true>(p, a->slot_dtype, vec, s) : launch_store_idx<F16T, false>(p, a->slot_dtype, vec, s);
    case FA_BF16: return fp8 ? launch_store_idx<BF16T, true>(p, a->slot_dtype, vec, s) : launch_store_idx<BF16T, false>(p, a->slot_dtype, vec, s);
    default: return fp8 ? launch_store_idx<F32T, true>(p, a->slot_dtype, vec, s) : launch_store_idx<F32T, false>(p, a->slot_dtype, vec, s);
  }
}

extern "C" int fa_append_kvcache(const fa_append_args* a, void* stream) {
  FA_REQUIRE(a != nullptr && a->lengths != nullptr, "fa_append_kvcache: null args/lengths");
  const int ndesc = a->kv[1].x ? 2 : 1;
  const int xdt = a->kv[0].x_dtype, cdt = a->kv[0].cache_dtype;
  for (int i = 0; i < ndesc; ++i) {
    const fa_store_desc& s = a->kv[i];
    FA_REQUIRE(s.x && s.cache, "fa_append_kvcache: null tensor %d", i);
    FA_REQUIRE(s.x_dtype == xdt && s.cache_dtype == cdt, "fa_append_kvcache: K and V must share dtypes");
    FA_REQUIRE(s.x_dtype == FA_F16 || s.x_dtype == FA_BF16 || s.x_dtype == FA_F32,
               "fa_append_kvcache: input dtype must be f16/bf16/f32");
    FA_REQUIRE(s.cache_dtype == s.x_dtype || s.cache_dtype == FA_E4M3,
               "fa_append_kvcache: cache dtype must match input or be E4M3");
    FA_REQUIRE(s.cache_dtype != FA_E4M3 || s.scale != nullptr, "fa_append_kvcache: E4M3 cache needs a scale");
  }
  FA_REQUIRE(a->page_size > 0, "fa_append_kvcache: bad page size");
  FA_REQUIRE(a->block_table == nullptr || a->table_cols > 0, "fa_append_kvcache: empty block table");
  int64_t work = 0;
  AppendParams p;
  for (int i = 0; i < 2; ++i) {
    p.d[i] = to_desc(a->kv[i < ndesc ? i : 0], 1);
    p.xb[i] = a->x_batch_stride[i < ndesc ? i : 0];
    const int64_t w = a->batch * a->new_tokens * p.d[i].heads * p.d[i].dim;
    work = w > work ? w : work;
  }
  if (work == 0) return FA_OK;
  p.lengths = a->lengths;
  p.batch_index = a->batch_index;
  p.table = a->block_table;
  p.batch = a->batch;
  p.new_tokens = a->new_tokens;
  p.page_size = a->page_size;
  p.num_blocks = a->num_blocks;
  p.table_rows = a->table_rows;
  p.table_cols = a->table_cols;
  p.ndesc = ndesc;
  int64_t blocks = fa_ceil_div(work, 256);
  if (blocks > 65535 * 8) blocks = 65535 * 8;
  dim3 grid((unsigned)blocks, (unsigned)ndesc);
  hipStream_t s = (hipStream_t)stream;
  const bool fp8 = cdt == FA_E4M3;
  switch (xdt) {
    case FA_F16:
      if (fp8) hipLaunchKernelGGL((append_kernel<F16T, true>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((append_kernel<F16T, false>), grid, dim3(256), 0, s, p);
      break;
    case FA_BF16:
      if (fp8) hipLaunchKernelGGL((append_kernel<BF16T, true>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((append_kernel<BF16T, false>), grid, dim3(256), 0, s, p);
      break;
    default:
      if (fp8) hipLaunchKernelGGL((append_kernel<F32T, true>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((append_kernel<F32T, false>), grid, dim3(256), 0, s, p);
      break;
  }
  return fa_check_launch("fa_append_kvcache");
}

extern "C" int fa_rotary(const fa_rotary_args* a, void* stream) {
  FA_REQUIRE(a && a->x && a->out && a->cos_table && a->sin_table && a->lengths, "fa_rotary: null argument");
  FA_REQUIRE(a->dtype == FA_F16 || a->dtype == FA_BF16 || a->dtype == FA_F32, "fa_rotary: dtype must be f16/bf16/f32");
  FA_REQUIRE(2 * a->half_rot <= a->dim, "fa_rotary: rotary dim exceeds head dim");
  RotaryParams p;
  p.x = a->x;
  p.out = a->out;
  p.cos_t = a->cos_table;
  p.sin_t = a->sin_table;
  p.lengths = a->lengths;
  p.batch = a->batch;
  p.seq = a->seq;
  p.heads = a->heads;
  p.dim = a->dim;
  p.half = a->half_rot;
  p.rows = a->table_rows;
  for (int i = 0; i < 4; ++i) p.xs[i] = a->x_stride[i];
  p.interleaved = a->interleaved;
  p.advance = a->advance;
  const int64_t total = p.batch * p.seq * p.heads * p.dim;
  if (total == 0) return FA_OK;
  int64_t blocks = fa_ceil_div(total, 256);
  if (blocks > 65535 * 8) blocks = 65535 * 8;
  hipStream_t s = (hipStream_t)stream;
  switch (a->dtype) {
    case FA_F16: hipLaunchKernelGGL((rotary_kernel<F16T>), dim3((unsigned)blocks), dim3(256), 0, s, p); break;
    case FA_BF16: hipLaunchKernelGGL((rotary_kernel<BF16T>), dim3((unsigned)blocks), dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL((rotary_kernel<F32T>), dim3((unsigned)blocks), dim3(256), 0, s, p); break;
  }
  return fa_check_launch("fa_rotary");
}
