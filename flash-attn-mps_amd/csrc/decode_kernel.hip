// Single-query split-KV decode over packed or paged K/V, plus the split merge.
//
// Semantics follow flash_attn_mps/_decode.py:40-99 and
// flash_attn_mps/kernels/attention_decode.metal:18-207: one query per request,
// keys [vis_begin, len) with vis_begin = len - window_left - 1 under a left
// window, q pre-scaled by softmax_scale * q_descale * k_descale, softcap on the
// scaled score, the sink seeding (max, sum) = (sink, 1) of split 0 only, the
// output multiplied by v_descale, fp32 partial states merged by log-sum-exp.
//
// gfx950 layout.  A workgroup (4 waves) owns one (request, group of GT query
// heads sharing a KV head, split of `span` keys).  Every 16-lane row of a wave
// owns one key at a time and spreads its head dimension over the 16 lanes,
// so each lane moves D/16 contiguous elements per key with 4..16-byte loads:
// a 256-byte bf16/FP8 head row is one fully coalesced 16-lane access.  A wave
// step covers 32 key positions (4 rows x 8 positions; 8 consecutive positions
// share one page when P % 8 == 0; 4 positions for 512-byte K+V row pairs)
// and issues all of its K and V loads before any arithmetic, which keeps
// 8-16 KiB per wave in flight for the HBM stream.
// Scores are reduced across the 16 lanes with DPP; each row keeps its own
// online-softmax state, combined across rows with lane shuffles and across
// waves through LDS at the end.  Math is exp2-based with log2(e) folded into q.
#include "attn_common.h"

namespace {

constexpr int DEC_THREADS = 256;
constexpr int DEC_PAGE_ALIGN = 8;   // paged K/V needs P % 8 == 0

// Positions per 16-lane row per step: 8, or 4 when a K+V row pair is wide
// enough that 8 of each in flight would exceed the register budget.
template <int KB, int VB>
struct DecodeRows {
  static constexpr int value = (KB + VB) / 4 * 8 > 96 ? 4 : 8;
};

template <int BYTES>
struct LoadChunk {
  static constexpr int value = BYTES % 16 == 0 ? 16 : BYTES % 8 == 0 ? 8 : 4;
};

template <int BYTES>
FA_DEV void load_words(const char* p, uint32_t (&w)[BYTES / 4]) {
  constexpr int C = LoadChunk<BYTES>::value;
#pragma unroll
  for (int c = 0; c < BYTES / C; ++c) {
    if constexpr (C == 16) {
      const uint4 v = *(const uint4*)(p + 16 * c);
      w[4 * c] = v.x; w[4 * c + 1] = v.y; w[4 * c + 2] = v.z; w[4 * c + 3] = v.w;
    } else if constexpr (C == 8) {
      const uint2 v = *(const uint2*)(p + 8 * c);
      w[2 * c] = v.x; w[2 * c + 1] = v.y;
    } else {
      w[c] = *(const uint32_t*)(p + 4 * c);
    }
  }
}

template <typename T, int N>
FA_DEV void words_to_f32(const uint32_t* w, float* f) {
  if constexpr (T::id == FA_BF16) {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else if constexpr (T::id == FA_F16) {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      f[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
      f[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
    }
  } else if constexpr (T::id == FA_E4M3) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
      f[4 * i] = lo[0]; f[4 * i + 1] = lo[1]; f[4 * i + 2] = hi[0]; f[4 * i + 3] = hi[1];
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) f[i] = __uint_as_float(w[i]);
  }
}

FA_DEV int decode_vis_begin(const fa_attn_args& a, int k_len) {
  return a.window_left >= 0 ? max(0, k_len - a.window_left - 1) : 0;
}

template <typename KT, typename VT, int D, int DV, int GT>
__global__ __launch_bounds__(DEC_THREADS, 2) void decode_kernel(const fa_attn_args a, const int span) {
  constexpr int EK = D / 16, EV = DV / 16;
  constexpr int KB = EK * KT::bytes, VB = EV * VT::bytes;
  constexpr int DEC_NT = DecodeRows<KB, VB>::value;
  constexpr int STEP = 4 * DEC_NT;   // positions per wave step
  static_assert(D % 16 == 0 && DV % 16 == 0 && KB % 4 == 0 && VB % 4 == 0, "decode tile shape");
  __shared__ float sm_m[4][GT], sm_l[4][GT];
  __shared__ float sm_acc[4][GT][DV];

  const int split = blockIdx.x;
  const int64_t b = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, rg = lane >> 4, l16 = lane & 15;
  const RequestInfo r = load_request(a, b);
  if (r.q_len != 1) return;
  const int group = (int)(a.heads_q / a.heads_k);
  const int h0 = blockIdx.y * GT;
  const int kh = h0 / group;
  const int vis_begin = decode_vis_begin(a, r.k_len);
  const int begin = vis_begin + split * span;
  const int end = min(r.k_len, begin + span);
  if (split > 0 && begin >= end) return;
  const int64_t tq = r.q_begin;
  const int S = a.num_splits;

  const bool cap = a.softcap > 0.0f;
  const float qscale = a.softmax_scale * descale_of(a.q_descale, a.q_descale_stride, b, kh) *
                       descale_of(a.k_descale, a.k_descale_stride, b, kh) * (cap ? 1.0f : LOG2E);
  const float vscale = descale_of(a.v_descale, a.v_descale_stride, b, kh);

  float q[GT][EK];
#pragma unroll
  for (int g = 0; g < GT; ++g)
#pragma unroll
    for (int e = 0; e < EK; ++e)
      q[g][e] = load_any(a.q, tq * a.q_stride[0] + (int64_t)(h0 + g) * a.q_stride[1] + (int64_t)(l16 * EK + e) * a.q_stride[2],
                         a.q_dtype) * qscale;

  float m[GT], l[GT], acc[GT][EV];
  const bool seed = a.sinks && split == 0 && wave == 0 && rg == 0;
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    m[g] = seed ? a.sinks[(int64_t)(h0 + g) * a.sink_stride] * LOG2E : -INFINITY;
    l[g] = seed ? 1.0f : 0.0f;
#pragma unroll
    for (int e = 0; e < EV; ++e) acc[g][e] = 0.0f;
  }

  const int64_t base = (int64_t)r.k_base + r.left;   // storage position of key 0
  const int64_t plo = base + begin, phi = base + end;
  const char* kc = (const char*)a.k;
  const char* vc = (const char*)a.v;
  const int64_t P = a.page_size;

  for (int64_t sb = (plo & ~(int64_t)(STEP - 1)) + STEP * wave; sb < phi; sb += 4 * STEP) {
    const int64_t rpos = sb + DEC_NT * rg;
    int64_t koff = 0, voff = 0;
    if (rpos + DEC_NT > plo && rpos < phi) {
      if (P) {
        const int64_t page = rpos / P;
        const int64_t blk = a.block_table[b * a.bt_stride[0] + page * a.bt_stride[1]];
        const int64_t in = rpos - page * P;
        koff = blk * a.k_stride[0] + in * a.k_stride[1] + (int64_t)kh * a.k_stride[2];
        voff = blk * a.v_stride[0] + in * a.v_stride[1] + (int64_t)kh * a.v_stride[2];
      } else {
        koff = rpos * a.k_stride[1] + (int64_t)kh * a.k_stride[2];
        voff = rpos * a.v_stride[1] + (int64_t)kh * a.v_stride[2];
      }
    }
    uint32_t kw[DEC_NT][KB / 4], vw[DEC_NT][VB / 4];
    bool ok[DEC_NT];
#pragma unroll
    for (int i = 0; i < DEC_NT; ++i) {
      ok[i] = rpos + i >= plo && rpos + i < phi;
      if (ok[i]) {
        load_words<KB>(kc + (koff + i * a.k_stride[1] + l16 * EK) * KT::bytes, kw[i]);
      } else {
#pragma unroll
        for (int w = 0; w < KB / 4; ++w) kw[i][w] = 0u;
      }
    }
#pragma unroll
    for (int i = 0; i < DEC_NT; ++i) {
      if (ok[i]) {
        load_words<VB>(vc + (voff + i * a.v_stride[1] + l16 * EV) * VT::bytes, vw[i]);
      } else {
#pragma unroll
        for (int w = 0; w < VB / 4; ++w) vw[i][w] = 0u;
      }
    }
    float s[GT][DEC_NT];
#pragma unroll
    for (int i = 0; i < DEC_NT; ++i) {
      float kf[EK];
      words_to_f32<KT, EK>(kw[i], kf);
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        float dot = 0.0f;
#pragma unroll
        for (int e = 0; e < EK; ++e) dot = fmaf(q[g][e], kf[e], dot);
        s[g][i] = dot;
      }
    }
#pragma unroll
    for (int g = 0; g < GT; ++g)
#pragma unroll
      for (int i = 0; i < DEC_NT; ++i) {
        float v = row16_sum(s[g][i]);
        if (cap) v = a.softcap * tanhf(v / a.softcap) * LOG2E;
        s[g][i] = ok[i] ? v : -INFINITY;
      }
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      float mx = s[g][0];
#pragma unroll
      for (int i = 1; i < DEC_NT; ++i) mx = fmaxf(mx, s[g][i]);
      const float m_new = fmaxf(m[g], mx);
      const float ref = m_new == -INFINITY ? 0.0f : m_new;
      const float f = fast_exp2(m[g] - ref);
      float sum = 0.0f;
#pragma unroll
      for (int i = 0; i < DEC_NT; ++i) {
        s[g][i] = fast_exp2(s[g][i] - ref);
        sum += s[g][i];
      }
      l[g] = l[g] * f + sum;
      m[g] = m_new;
#pragma unroll
      for (int e = 0; e < EV; ++e) acc[g][e] *= f;
    }
#pragma unroll
    for (int i = 0; i < DEC_NT; ++i) {
      float vf[EV];
      words_to_f32<VT, EV>(vw[i], vf);
#pragma unroll
      for (int g = 0; g < GT; ++g)
#pragma unroll
        for (int e = 0; e < EV; ++e) acc[g][e] = fmaf(s[g][i], vf[e], acc[g][e]);
    }
  }

  // Combine the four 16-lane rows of the wave (same l16 <-> same dims).
#pragma unroll
  for (int g = 0; g < GT; ++g) {
#pragma unroll
    for (int mask = 16; mask <= 32; mask <<= 1) {
      const float mo = shfl_xor_f(m[g], mask);
      const float lo = shfl_xor_f(l[g], mask);
      const float mn = fmaxf(m[g], mo);
      const float ref = mn == -INFINITY ? 0.0f : mn;
      const float fa = fast_exp2(m[g] - ref), fb = fast_exp2(mo - ref);
      l[g] = l[g] * fa + lo * fb;
#pragma unroll
      for (int e = 0; e < EV; ++e) acc[g][e] = acc[g][e] * fa + shfl_xor_f(acc[g][e], mask) * fb;
      m[g] = mn;
    }
  }
  if (rg == 0) {
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      if (l16 == 0) {
        sm_m[wave][g] = m[g];
        sm_l[wave][g] = l[g];
      }
#pragma unroll
      for (int e = 0; e < EV; ++e) sm_acc[wave][g][l16 * EV + e] = acc[g][e];
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < GT * DV; idx += DEC_THREADS) {
    const int g = idx / DV, d = idx - g * DV;
    float M = sm_m[0][g];
#pragma unroll
    for (int w = 1; w < 4; ++w) M = fmaxf(M, sm_m[w][g]);
    const float ref = M == -INFINITY ? 0.0f : M;
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = fast_exp2(sm_m[w][g] - ref);
      L += sm_l[w][g] * f;
      O += sm_acc[w][g][d] * f;
    }
    const float norm = L > 0.0f ? vscale / L : 0.0f;
    const float lse = L > 0.0f ? M * LN2 + logf(L) : -INFINITY;
    const int h = h0 + g;
    if (S == 1) {
      store_any(a.out, tq * a.out_stride[0] + (int64_t)h * a.out_stride[1] + (int64_t)d * a.out_stride[2], a.out_dtype,
                O * norm);
      if (d == 0) a.lse[(int64_t)h * a.lse_stride[0] + tq * a.lse_stride[1]] = lse;
    } else {
      const int64_t row = (b * a.heads_q + h) * S + split;
      a.partial_out[row * DV + d] = O * norm;
      if (d == 0) a.partial_lse[row] = lse;
    }
  }
}

// One wavefront merges the valid splits of one (request, head) row into the
// caller's output.  Splits past the request's last key were never written.
__global__ __launch_bounds__(256) void decode_merge_kernel(const fa_attn_args a, const int span) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= a.batch * a.heads_q) return;
  const int64_t b = row / a.heads_q, h = row - b * a.heads_q;
  const RequestInfo r = load_request(a, b);
  if (r.q_len != 1) return;
  const int S = a.num_splits;
  const int n = r.k_len - decode_vis_begin(a, r.k_len);
  const int nv = n > 0 ? min(S, (n + span - 1) / span) : 1;
  const float* plse = a.partial_lse + row * S;
  const float* po = a.partial_out + row * S * a.head_dim_v;
  float peak = -INFINITY;
  for (int s = lane; s < nv; s += 64) peak = fmaxf(peak, plse[s]);
  peak = wave_max(peak);
  const float ref = peak == -INFINITY ? 0.0f : peak;
  float denom = 0.0f;
  for (int s = lane; s < nv; s += 64) denom += expf(plse[s] - ref);
  denom = wave_sum(denom);
  const int64_t tq = r.q_begin;
  for (int d = lane; d < a.head_dim_v; d += 64) {
    float v = 0.0f;
    for (int s = 0; s < nv; ++s) {
      const float w = expf(plse[s] - ref);
      if (w > 0.0f) v = fmaf(w, po[(int64_t)s * a.head_dim_v + d], v);
    }
    store_any(a.out, tq * a.out_stride[0] + h * a.out_stride[1] + (int64_t)d * a.out_stride[2], a.out_dtype,
              denom > 0.0f ? v / denom : 0.0f);
  }
  if (lane == 0) a.lse[h * a.lse_stride[0] + tq * a.lse_stride[1]] = denom > 0.0f ? peak + logf(denom) : -INFINITY;
}

using DecodeKernel = void (*)(fa_attn_args, int);

template <typename KT, typename VT, int D, int DV>
DecodeKernel pick_group(int gt) {
  switch (gt) {
    case 4: if constexpr (4 * (D + DV) <= 64 * 16) return decode_kernel<KT, VT, D, DV, 4>; else return nullptr;
    case 2: if constexpr (2 * (D + DV) <= 64 * 16) return decode_kernel<KT, VT, D, DV, 2>; else return nullptr;
    case 1: return decode_kernel<KT, VT, D, DV, 1>;
    default: return nullptr;
  }
}

template <typename KT, typename VT>
DecodeKernel pick_dims(int64_t d, int64_t dv, int gt) {
  if (d == 64 && dv == 64) return pick_group<KT, VT, 64, 64>(gt);
  if (d == 128 && dv == 128) return pick_group<KT, VT, 128, 128>(gt);
  if (d == 192 && dv == 128) return pick_group<KT, VT, 192, 128>(gt);
  if (d == 256 && dv == 256) return pick_group<KT, VT, 256, 256>(gt);
  return nullptr;
}

int elem_size(int dt) { return dt == FA_F32 ? 4 : dt == FA_E4M3 ? 1 : 2; }

// Largest query-head group sharing one KV head that keeps q + accumulators
// within 64 fp32 registers per lane.
int decode_group_tile(const fa_attn_args& a) {
  const int64_t group = a.heads_q / a.heads_k;
  const int64_t per = (a.head_dim_qk + a.head_dim_v) / 16;
  for (int gt = 4; gt >= 1; gt >>= 1)
    if (group % gt == 0 && gt * per <= 64) return gt;
  return 1;
}

bool chunk_aligned(const void* p, const int64_t* st, int nstrides, int esz, int bytes_per_lane) {
  const int c = bytes_per_lane % 16 == 0 ? 16 : bytes_per_lane % 8 == 0 ? 8 : 4;
  if (((uintptr_t)p) % c) return false;
  for (int i = 0; i < nstrides; ++i)
    if ((st[i] * esz) % c) return false;
  return true;
}

DecodeKernel select_decode(const fa_attn_args& a, int* gt_out) {
  if (a.k_dtype != a.v_dtype) return nullptr;
  if (a.mask_kind != 0 || a.alibi) return nullptr;
  if (a.page_size && a.page_size % DEC_PAGE_ALIGN) return nullptr;
  if (a.k_stride[3] != 1 || a.v_stride[3] != 1) return nullptr;
  const int esz = elem_size(a.k_dtype);
  if ((a.head_dim_qk / 16) * esz % 4 || (a.head_dim_v / 16) * esz % 4) return nullptr;
  if (!chunk_aligned(a.k, a.k_stride, 3, esz, (int)(a.head_dim_qk / 16) * esz)) return nullptr;
  if (!chunk_aligned(a.v, a.v_stride, 3, esz, (int)(a.head_dim_v / 16) * esz)) return nullptr;
  const int gt = decode_group_tile(a);
  *gt_out = gt;
  switch (a.k_dtype) {
    case FA_BF16: return pick_dims<BF16T, BF16T>(a.head_dim_qk, a.head_dim_v, gt);
    case FA_F16: return pick_dims<F16T, F16T>(a.head_dim_qk, a.head_dim_v, gt);
    case FA_E4M3: return pick_dims<E4M3T, E4M3T>(a.head_dim_qk, a.head_dim_v, gt);
    default: return nullptr;
  }
}

}  // namespace

extern "C" int fa_decode_supported(const fa_attn_args* a) {
  if (!a) return 0;
  int gt = 0;
  return select_decode(*a, &gt) != nullptr;
}

extern "C" int fa_decode_fwd(const fa_attn_args* a, void* stream) {
  int rc = fa_validate_attn(a, "fa_decode_fwd");
  if (rc) return rc;
  int gt = 1;
  const DecodeKernel kern = select_decode(*a, &gt);
  if (!kern) {
    fa_set_error("fa_decode_fwd: unsupported dtype/head-dim/stride combination");
    return FA_ERR_UNSUPPORTED;
  }
  if (a->total_q == 0) return FA_OK;
  FA_REQUIRE(a->split_span >= 1, "fa_decode_fwd: split_span must be positive");
  FA_REQUIRE(a->num_splits == 1 || (a->partial_out && a->partial_lse), "fa_decode_fwd: splits need partial buffers");
  FA_REQUIRE(a->batch <= 65535, "fa_decode_fwd: batch exceeds the grid limit");
  const int64_t head_groups = a->heads_q / gt;
  FA_REQUIRE(head_groups <= 65535, "fa_decode_fwd: too many heads");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)a->num_splits, (unsigned)head_groups, (unsigned)a->batch);
  hipLaunchKernelGGL(kern, grid, dim3(DEC_THREADS), 0, s, *a, (int)a->split_span);
  rc = fa_check_launch("fa_decode_fwd");
  if (rc || a->num_splits == 1) return rc;
  const int64_t rows = a->batch * a->heads_q;
  hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)fa_ceil_div(rows, 4)), dim3(256), 0, s, *a, (int)a->split_span);
  return fa_check_launch("fa_decode_fwd merge");
}
