// Generic fused attention: every feature of the reference's tiled/vector
// kernels (flash_attn_mps/kernels/attention.metal:60-248) -- paged or packed
// K/V, left padding, static or per-request causality, windows, ALiBi, sinks,
// q/k/v descales, mask kinds 1/2, softcap, split-KV partials, head dims
// 1..512 (Dqk != Dv allowed), fp16/bf16/fp32/E4M3 inputs and any strides.
//
// One wavefront owns one (query row, head, split).  Each pass scores 64 keys
// at once (one key per lane, dot product over the head dimension), updates
// the running max/sum with wave reductions, then accumulates P*V with lanes
// owning output dimensions.  A row's result depends only on that row's data
// and its split range, never on the rest of the batch, so num_splits == 1 is
// batch-invariant (flash_attn_mps/tests/test_vllm.py:152-159).
#include "attn_common.h"

namespace {

constexpr int GEN_WAVES = 4;
constexpr int GEN_MAX_D = 512;

template <typename KT, typename VT>
__global__ __launch_bounds__(256) void attn_generic_kernel(const fa_attn_args a) {
  __shared__ float q_smem[GEN_WAVES][GEN_MAX_D];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t S = a.num_splits;
  const int64_t b = blockIdx.z / S, split = blockIdx.z - (blockIdx.z / S) * S;
  const int h = blockIdx.y;
  const int qi = blockIdx.x * GEN_WAVES + wave;
  const int group = (int)(a.heads_q / a.heads_k);
  const int kh = h / group;
  const RequestInfo r = load_request(a, b);
  const bool active = qi < r.q_len;
  const int64_t tq = (int64_t)r.q_begin + qi;
  const int Dq = (int)a.head_dim_qk, Dv = (int)a.head_dim_v;
  if (active)
    for (int d = lane; d < Dq; d += 64)
      q_smem[wave][d] = load_any(a.q, tq * a.q_stride[0] + (int64_t)h * a.q_stride[1] + d * a.q_stride[2], a.q_dtype);
  __syncthreads();
  if (!active) return;

  const float scale = a.softmax_scale * descale_of(a.q_descale, a.q_descale_stride, b, kh) *
                      descale_of(a.k_descale, a.k_descale_stride, b, kh);
  const float vscale = descale_of(a.v_descale, a.v_descale_stride, b, kh);
  const float slope = a.alibi ? a.alibi[b * a.alibi_stride[0] + (int64_t)h * a.alibi_stride[1]] : 0.0f;
  const float sink = (a.sinks && split == 0) ? a.sinks[(int64_t)h * a.sink_stride] : -INFINITY;
  const int q_abs = qi + r.k_len - r.q_len;

  int begin = (int)((int64_t)r.k_len * split / S);
  int end = (int)((int64_t)r.k_len * (split + 1) / S);
  if (a.mask_kind == 0) {
    if (r.causal) end = min(end, q_abs + 1);
    if (a.window_left >= 0) begin = max(begin, q_abs - a.window_left);
    if (a.window_right >= 0) end = min(end, q_abs + a.window_right + 1);
  }

  float m = sink;
  float l = sink > -INFINITY ? 1.0f : 0.0f;
  float acc[GEN_MAX_D / 64];
#pragma unroll
  for (int i = 0; i < GEN_MAX_D / 64; ++i) acc[i] = 0.0f;
  const float* qrow = q_smem[wave];

  for (int t0 = begin; t0 < end; t0 += 64) {
    const int t = t0 + lane;
    const bool valid = t < end && key_allowed(a, b, t, q_abs, tq, r.causal);
    float s = -INFINITY;
    if (valid) {
      const int64_t off = kv_offset(a, a.k_stride, b, r, t, kh);
      float dot = 0.0f;
      for (int d = 0; d < Dq; ++d) dot = fmaf(qrow[d], load_elem<KT>(a.k, off + d * a.k_stride[3]), dot);
      s = dot * scale;
      if (a.softcap > 0.0f) s = a.softcap * tanhf(s / a.softcap);
      s -= slope * (float)abs(q_abs - t);
    }
    const float m_new = fmaxf(m, wave_max(s));
    if (m_new == -INFINITY) continue;
    const float factor = expf(m - m_new);
    const float p = valid ? expf(s - m_new) : 0.0f;
    l = l * factor + wave_sum(p);
#pragma unroll
    for (int i = 0; i < GEN_MAX_D / 64; ++i) acc[i] *= factor;
    const int n = min(64, end - t0);
    for (int j = 0; j < n; ++j) {
      const float pj = readlane_f(p, j);
      if (pj == 0.0f) continue;
      const int64_t voff = kv_offset(a, a.v_stride, b, r, t0 + j, kh);
#pragma unroll
      for (int i = 0; i < GEN_MAX_D / 64; ++i) {
        const int e = lane + 64 * i;
        if (e < Dv) acc[i] = fmaf(pj, load_elem<VT>(a.v, voff + e * a.v_stride[3]), acc[i]);
      }
    }
    m = m_new;
  }

  const float norm = l > 0.0f ? vscale / l : 0.0f;
  const float lse = l > 0.0f ? m + logf(l) : -INFINITY;
  if (S == 1) {
#pragma unroll
    for (int i = 0; i < GEN_MAX_D / 64; ++i) {
      const int e = lane + 64 * i;
      if (e < Dv)
        store_any(a.out, tq * a.out_stride[0] + (int64_t)h * a.out_stride[1] + e * a.out_stride[2], a.out_dtype,
                  acc[i] * norm);
    }
    if (lane == 0) a.lse[(int64_t)h * a.lse_stride[0] + tq * a.lse_stride[1]] = lse;
  } else {
    float* po = a.partial_out + ((split * a.total_q + tq) * a.heads_q + h) * (int64_t)Dv;
#pragma unroll
    for (int i = 0; i < GEN_MAX_D / 64; ++i) {
      const int e = lane + 64 * i;
      if (e < Dv) po[e] = acc[i] * norm;
    }
    if (lane == 0) a.partial_lse[(split * a.heads_q + h) * a.total_q + tq] = lse;
  }
}

template <typename KT>
int launch_generic_v(const fa_attn_args& a, dim3 grid, hipStream_t s) {
  switch (a.v_dtype) {
    case FA_F16: hipLaunchKernelGGL((attn_generic_kernel<KT, F16T>), grid, dim3(256), 0, s, a); break;
    case FA_BF16: hipLaunchKernelGGL((attn_generic_kernel<KT, BF16T>), grid, dim3(256), 0, s, a); break;
    case FA_E4M3: hipLaunchKernelGGL((attn_generic_kernel<KT, E4M3T>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((attn_generic_kernel<KT, F32T>), grid, dim3(256), 0, s, a); break;
  }
  return fa_check_launch("fa_attn_fwd");
}

bool valid_dtype(int d) { return d == FA_F16 || d == FA_BF16 || d == FA_F32 || d == FA_E4M3; }

}  // namespace

int fa_validate_attn(const fa_attn_args* a, const char* who) {
  // K/V may be empty (a null data pointer) when every request has zero keys.
  FA_REQUIRE(a && a->q && a->out && a->lse && a->cu_seqlens_q, "%s: null tensor", who);
  FA_REQUIRE(valid_dtype(a->q_dtype) && valid_dtype(a->k_dtype) && valid_dtype(a->v_dtype), "%s: bad input dtype", who);
  FA_REQUIRE(a->out_dtype == FA_F16 || a->out_dtype == FA_BF16 || a->out_dtype == FA_F32, "%s: bad output dtype", who);
  FA_REQUIRE(a->head_dim_qk >= 1 && a->head_dim_qk <= 512 && a->head_dim_v >= 1 && a->head_dim_v <= 512,
             "%s: head dims must be in 1..512", who);
  FA_REQUIRE(a->heads_k >= 1 && a->heads_q >= 1 && a->heads_q % a->heads_k == 0, "%s: Hq must be a multiple of Hkv", who);
  FA_REQUIRE(a->batch >= 1, "%s: batch must be positive", who);
  FA_REQUIRE(a->cu_seqlens_k || a->seqused_k, "%s: need cu_seqlens_k or seqused_k", who);
  FA_REQUIRE(a->page_size == 0 || a->block_table, "%s: paged K/V needs a block table", who);
  FA_REQUIRE(a->mask_kind == 0 || a->mask_kind == 1 || a->mask_kind == 2, "%s: bad mask kind", who);
  FA_REQUIRE(a->mask_kind != 1 || a->mask_ranges, "%s: mask kind 1 needs ranges", who);
  FA_REQUIRE(a->mask_kind != 2 || (a->mask_prefix && a->mask_window_len), "%s: mask kind 2 needs prefix/window", who);
  FA_REQUIRE(a->num_splits >= 1, "%s: num_splits must be >= 1", who);
  return FA_OK;
}

extern "C" int fa_attn_fwd(const fa_attn_args* a, void* stream) {
  int rc = fa_validate_attn(a, "fa_attn_fwd");
  if (rc) return rc;
  if (a->total_q == 0) return FA_OK;
  FA_REQUIRE(a->num_splits == 1 || (a->partial_out && a->partial_lse), "fa_attn_fwd: splits need partial buffers");
  FA_REQUIRE(a->max_seqlen_q >= 1, "fa_attn_fwd: max_seqlen_q must be positive");
  FA_REQUIRE(a->batch * a->num_splits <= 65535, "fa_attn_fwd: batch*splits exceeds the grid limit");
  FA_REQUIRE(a->heads_q <= 65535, "fa_attn_fwd: too many heads");
  const dim3 grid((unsigned)fa_ceil_div(a->max_seqlen_q, GEN_WAVES), (unsigned)a->heads_q,
                  (unsigned)(a->batch * a->num_splits));
  hipStream_t s = (hipStream_t)stream;
  switch (a->k_dtype) {
    case FA_F16: rc = launch_generic_v<F16T>(*a, grid, s); break;
    case FA_BF16: rc = launch_generic_v<BF16T>(*a, grid, s); break;
    case FA_E4M3: rc = launch_generic_v<E4M3T>(*a, grid, s); break;
    default: rc = launch_generic_v<F32T>(*a, grid, s); break;
  }
  if (rc || a->num_splits == 1) return rc;
  fa_merge_partials_args m;
  m.partial = a->partial_out;
  m.partial_lse = a->partial_lse;
  m.out = a->out;
  m.lse = a->lse;
  m.partial_dtype = FA_F32;
  m.out_dtype = a->out_dtype;
  m.splits = a->num_splits;
  m.tokens = a->total_q;
  m.heads = a->heads_q;
  m.dim = a->head_dim_v;
  m.partial_stride[0] = a->total_q * a->heads_q * a->head_dim_v;
  m.partial_stride[1] = a->heads_q * a->head_dim_v;
  m.partial_stride[2] = a->head_dim_v;
  m.partial_stride[3] = 1;
  m.partial_lse_stride[0] = a->heads_q * a->total_q;
  m.partial_lse_stride[1] = a->total_q;
  m.partial_lse_stride[2] = 1;
  for (int i = 0; i < 3; ++i) m.out_stride[i] = a->out_stride[i];
  for (int i = 0; i < 2; ++i) m.lse_stride[i] = a->lse_stride[i];
  return fa_merge_partials(&m, stream);
}
