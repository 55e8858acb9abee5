// Split-KV decode: the merge kernel, kernel selection and the C-ABI entry
// points fa_decode_supported / fa_decode_fwd (flash_attn_mps/_decode.py:40-99)
// and fa_decode_fwd_noalloc (no reference counterpart).  The decode kernel
// itself is in decode_kernel.h; its variants are instantiated in
// decode_inst_*.hip.
#include <mutex>

#include "decode_kernel.h"

// Split partials of fa_decode_fwd_noalloc, one copy per GPU, held until the
// process ends.  In host code this name is only a stand-in for the symbol:
// the device address comes from hipGetSymbolAddress (scratch_of_device) and
// is the only thing ever handed to a kernel.
static __device__ __align__(256) float scratch[FA_DECODE_SCRATCH_BYTES / sizeof(float)];

namespace {

using namespace fa_decode;

// One wavefront merges the valid splits of one (request, token, head) row
// into the caller's output.  Splits past the request's last key were never
// written.
// Split weights exp(lse_s - max) are computed once, 64 splits at a time (split
// s0 + j on lane j), and broadcast with readlane; every lane accumulates the
// dims lane, lane + 64, ... (DIMS of them, Dv <= 64 DIMS) so each partial row
// is one coalesced read.  The first GROUP partial rows are loaded together
// with the LSEs, before the weights are known, so a row with at most GROUP
// splits costs one round trip to memory before its store; further splits
// follow GROUP at a time.  Splits are added in order, whatever GROUP is.
//
// Rows are (request, token, head) with max_seqlen_q tokens per request (the
// multi-token GQA decode) or one; rows past a request's tokens, and requests
// with more tokens than that, do nothing.
template <int DIMS, int GROUP>
__global__ __launch_bounds__(256) void decode_merge_kernel(const fa_attn_args a, const int span) {
  static_assert(GROUP <= 64, "the first group's weights sit on lanes 0 .. GROUP - 1");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ntok = a.max_seqlen_q > 1 ? (int)a.max_seqlen_q : 1;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= a.batch * ntok * a.heads_q) return;
  const int64_t b = row / (ntok * a.heads_q), bt = row / a.heads_q, h = row - bt * a.heads_q;
  const int t = (int)(bt - b * ntok);
  const RequestInfo r = load_request(a, b);
  if (r.q_len < 1 || r.q_len > ntok || t >= r.q_len) return;   // the decode kernel skipped the request
  const int S = a.num_splits;
  const int DV = (int)a.head_dim_v;
  const int n = r.k_len - decode_vis_begin(a, r.k_len, r.q_len);
  const int nv = n > 0 ? min(S, (n + span - 1) / span) : 1;
  // Partial outputs [batch][S][ntok][Hq][Dv]: this row's splits are pitch
  // floats apart; LSEs [batch][ntok][Hq][S] contiguous.
  const int64_t rows_b = (int64_t)ntok * a.heads_q, pitch = rows_b * DV;
  const float* plse = a.partial_lse + row * S;
  const float* po = a.partial_out + (b * S * rows_b + (row - b * rows_b)) * DV;
  // A zero-weight split (empty, its partial never written) is read like the
  // others but dropped by a select, so its contents never reach the sum.
  float x0[GROUP][DIMS];
#pragma unroll
  for (int u = 0; u < GROUP; ++u)
#pragma unroll
    for (int k = 0; k < DIMS; ++k)
      x0[u][k] = u < nv && lane + 64 * k < DV ? po[(int64_t)u * pitch + lane + 64 * k] : 0.0f;
  const float lse0 = lane < nv ? plse[lane] : -INFINITY;
  float peak = lse0;
  for (int s = lane + 64; s < nv; s += 64) peak = fmaxf(peak, plse[s]);
  peak = wave_max(peak);
  const float ref = peak == -INFINITY ? 0.0f : peak;
  float acc[DIMS];
#pragma unroll
  for (int k = 0; k < DIMS; ++k) acc[k] = 0.0f;
  float w = lane < nv ? expf(lse0 - ref) : 0.0f;
  float denom = w;
#pragma unroll
  for (int u = 0; u < GROUP; ++u) {
    const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), u));
#pragma unroll
    for (int k = 0; k < DIMS; ++k) acc[k] = ws > 0.0f ? fmaf(ws, x0[u][k], acc[k]) : acc[k];
  }
  for (int s0 = 0; s0 < nv; s0 += 64) {
    if (s0) {
      w = s0 + lane < nv ? expf(plse[s0 + lane] - ref) : 0.0f;
      denom += w;
    }
    const int cnt = min(64, nv - s0);
    int j = s0 ? 0 : GROUP;
    for (; j + GROUP <= cnt; j += GROUP) {
      float ws[GROUP], x[GROUP][DIMS];
#pragma unroll
      for (int u = 0; u < GROUP; ++u) {
        ws[u] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j + u));
        const float* src = po + (int64_t)(s0 + j + u) * pitch;
#pragma unroll
        for (int k = 0; k < DIMS; ++k) x[u][k] = lane + 64 * k < DV ? src[lane + 64 * k] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < GROUP; ++u)
#pragma unroll
        for (int k = 0; k < DIMS; ++k) acc[k] = ws[u] > 0.0f ? fmaf(ws[u], x[u][k], acc[k]) : acc[k];
    }
    for (; j < cnt; ++j) {
      const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
      if (ws > 0.0f) {   // zero-weight splits are never read
        const float* src = po + (int64_t)(s0 + j) * pitch;
#pragma unroll
        for (int k = 0; k < DIMS; ++k)
          if (lane + 64 * k < DV) acc[k] = fmaf(ws, src[lane + 64 * k], acc[k]);
      }
    }
  }
  denom = wave_sum(denom);
  const int64_t tq = r.q_begin + t;
  const float inv = denom > 0.0f ? 1.0f / denom : 0.0f;
#pragma unroll
  for (int k = 0; k < DIMS; ++k) {
    const int d = lane + 64 * k;
    if (d < DV)
      store_any(a.out, tq * a.out_stride[0] + h * a.out_stride[1] + (int64_t)d * a.out_stride[2], a.out_dtype,
                acc[k] * inv);
  }
  if (lane == 0) a.lse[h * a.lse_stride[0] + tq * a.lse_stride[1]] = denom > 0.0f ? peak + logf(denom) : -INFINITY;
}

int elem_size(int dt) { return dt == FA_F32 ? 4 : dt == FA_E4M3 ? 1 : 2; }

// Most keys one request can see: max_seqlen_k, clipped by a left window
// (the query sits at the last key, so it sees window_left + 1 keys).
int64_t decode_visible_max(const fa_attn_args& a) {
  const int64_t m = a.max_seqlen_k > 0 ? a.max_seqlen_k : 0;
  const int64_t q = a.max_seqlen_q > 1 ? a.max_seqlen_q : 1;   // the first row sees window_left + q keys
  return a.window_left >= 0 && a.window_left + q < m ? a.window_left + q : m;
}

// Query heads per workgroup (GT).  Every workgroup of a KV head reads it
// again, so GT is the smallest power of two that reaches the fewest
// workgroups per KV head, ceil(group / gmax), where gmax keeps q +
// accumulators within 64 fp32 registers per lane, or 128 for 128-dim tiles
// (GT = 8: Hq/Hkv = 64/8 at d128 went 3.5 -> 4.4 TB/s; 64-dim tiles at 8
// halve the occupancy and run 15% slower).  A group that GT does not divide
// ends in a partial tile.
int decode_group_tile(const fa_attn_args& a) {
  const int64_t group = a.heads_q / a.heads_k;
  const int64_t per = (decode_tile_dim(a.head_dim_qk) + decode_tile_dim(a.head_dim_v)) / 16;
  int gmax = per == 16 ? 8 : 1;
  while (gmax < 4 && 2 * gmax * per <= 64) gmax *= 2;
  const int64_t tiles = (group + gmax - 1) / gmax;
  int gt = 1;
  while ((group + gt - 1) / gt > tiles) gt *= 2;
  return gt;
}

// KV heads per VALU-decode workgroup: 2 (decode_kernel PK = 2) when two
// neighbouring heads' rows sit next to each other in every key row (head
// stride = the head dim, rows of two heads or more), with 8 KV heads or
// more and no ALiBi, for E4M3 d128 (groups of 1-2: 128-byte head rows, read
// as 256-byte runs) and 16-bit 192/128 (groups of 1).  Measured in one
// process against the unpaired kernel on the same caches, calls alternated
// (64 requests of U[512, 32768] keys): E4M3 d128 16/8 5.34 -> 5.69 TB/s, 8/8
// 5.43 -> 5.95, 16/16 5.63 -> 6.29; config 5 (192/128, 16/16, beside the
// chunk prefill) 1743 -> 1694 us.  Rows of 256 bytes or more gain nothing
// and lose a little: 16-bit d128 16/8 6.20 -> 6.04, 16/16 6.38 -> 6.42, d256
// 16/16 6.36 -> 6.29, config 4 (E4M3 d256) 317 -> 325 us.  One split per
// request (the fixed-order route) keeps one head per workgroup: there the
// grid is one workgroup per request and head, and halving it made config
// 5's fixed-order call slower (1738 -> 1784 us).
int valu_pair(const fa_attn_args& a) {
  const int64_t dq = a.head_dim_qk, dv = a.head_dim_v, group = a.heads_q / a.heads_k;
  if (a.num_splits == 1) return 1;
  const bool e4m3_128 = a.k_dtype == FA_E4M3 && dq == 128 && dv == 128;
  const bool diffkv = a.k_dtype != FA_E4M3 && dq == 192 && dv == 128;
  if (a.alibi || !(e4m3_128 || diffkv)) return 1;
  if (a.heads_k % 2 || a.k_stride[2] != dq || a.v_stride[2] != dv || a.k_stride[1] < 2 * dq || a.v_stride[1] < 2 * dv)
    return 1;
  if (a.heads_k < 8) return 1;
  return group <= (diffkv ? 1 : 2) ? 2 : 1;
}

bool chunk_aligned(const void* p, const int64_t* st, int nstrides, int esz, int bytes_per_lane) {
  const int c = bytes_per_lane % 16 == 0 ? 16 : bytes_per_lane % 8 == 0 ? 8 : 4;
  if (((uintptr_t)p) % c) return false;
  for (int i = 0; i < nstrides; ++i)
    if ((st[i] * esz) % c) return false;
  return true;
}

DecodeKernel select_decode(const fa_attn_args& a, int* gt_out) {
  // The head-group arithmetic below divides by heads_k.
  if (a.heads_k < 1 || a.heads_q < 1 || a.heads_q % a.heads_k) return nullptr;
  if (a.max_seqlen_q > 1) return nullptr;   // one query row per request
  if (a.k_dtype != a.v_dtype) return nullptr;
  if (a.mask_kind != 0) return nullptr;
  if (a.page_size && a.page_size % DEC_PAGE_ALIGN) return nullptr;
  // Page and row strides are 32-bit byte counts in the kernel's addressing.
  for (int i = 0; i < 3; ++i)
    if (a.k_stride[i] < 0 || a.v_stride[i] < 0 || a.k_stride[i] * elem_size(a.k_dtype) >= (1ll << 32) ||
        a.v_stride[i] * elem_size(a.v_dtype) >= (1ll << 32))
      return nullptr;
  if (a.k_stride[3] != 1 || a.v_stride[3] != 1) return nullptr;
  const int esz = elem_size(a.k_dtype);
  // Lane chunks are tile dims / 16 elements (the tile may pad the head dim).
  const int64_t tq = decode_tile_dim(a.head_dim_qk), tv = decode_tile_dim(a.head_dim_v);
  if (!tq || !tv) return nullptr;
  if ((tq / 16) * esz % 4 || (tv / 16) * esz % 4) return nullptr;
  if (!chunk_aligned(a.k, a.k_stride, 3, esz, (int)(tq / 16) * esz)) return nullptr;
  if (!chunk_aligned(a.v, a.v_stride, 3, esz, (int)(tv / 16) * esz)) return nullptr;
  // Q.K runs on 16-bit pairs of the query's type: 16-bit K must match it,
  // FP8 K widens exactly to either.
  if (a.q_dtype != FA_BF16 && a.q_dtype != FA_F16) return nullptr;
  if (a.q_stride[2] == 1 && !chunk_aligned(a.q, a.q_stride, 2, 2, (int)(tq / 16) * 2)) return nullptr;
  const int pk = valu_pair(a);
  const int gt = pk == 2 ? 2 * (int)(a.heads_q / a.heads_k) : decode_group_tile(a);
  *gt_out = gt;
  const bool qbf = a.q_dtype == FA_BF16, cap = a.softcap > 0.0f, alibi = a.alibi != nullptr;
  const int64_t dq = a.head_dim_qk, dv = a.head_dim_v;
  switch (a.k_dtype) {
    case FA_BF16: return qbf ? pick_decode_bf16(dq, dv, gt, cap, alibi, pk) : nullptr;
    case FA_F16: return qbf ? nullptr : pick_decode_f16(dq, dv, gt, cap, alibi, pk);
    case FA_E4M3:
      return qbf ? pick_decode_fp8_bf16(dq, dv, gt, cap, alibi, pk) : pick_decode_fp8_f16(dq, dv, gt, cap, alibi, pk);
    default: return nullptr;
  }
}

// Workgroups per (request, split): KV heads x head tiles of the kernel that
// runs (32 / max_seqlen_q query heads for the matrix-core GQA kernel, GT for
// the VALU one); either kernel may take KV heads in pairs.
int64_t decode_head_groups(const fa_attn_args& a, int gt) {
  const int64_t group = a.heads_q / a.heads_k;
  const int64_t ntok = a.max_seqlen_q > 1 ? a.max_seqlen_q : 1;
  const GqaChoice gqa = pick_decode_gqa(a);
  if (gqa.kern) return a.heads_k / gqa.pack * fa_ceil_div(gqa.pack * group, 32 / ntok);
  const int pk = valu_pair(a);
  return a.heads_k / pk * fa_ceil_div(pk * group, gt);
}

}  // namespace

extern "C" int fa_decode_supported(const fa_attn_args* a) {
  if (!a) return 0;
  if (pick_decode_gqa(*a).kern) return 1;
  int gt = 0;
  return select_decode(*a, &gt) != nullptr;
}

namespace {

// Partial rows: [batch][max_seqlen_q][Hq] (outputs [batch][splits][rows][Dv],
// LSEs [batch][rows][splits]).
int64_t partial_rows(const fa_attn_args& a) {
  return a.batch * (a.max_seqlen_q > 1 ? a.max_seqlen_q : 1) * a.heads_q;
}

// Launch the decode kernel (and the merge when there are several splits) for
// arguments that passed fa_validate_attn.
int decode_launch(const fa_attn_args* a, void* stream, const char* who) {
  int gt = 1;
  const GqaChoice gqa = pick_decode_gqa(*a);
  const DecodeKernel kern = gqa.kern ? gqa.kern : select_decode(*a, &gt);
  if (!kern) {
    fa_set_error("%s: unsupported dtype/head-dim/stride combination", who);
    return FA_ERR_UNSUPPORTED;
  }
  if (a->total_q == 0) return FA_OK;
  FA_REQUIRE(a->split_span >= 1 && a->num_splits >= 1, "%s: num_splits and split_span must be positive", who);
  // Keys past num_splits * split_span would be dropped without a trace.
  FA_REQUIRE((int64_t)a->num_splits * a->split_span >= decode_visible_max(*a),
             "%s: num_splits * split_span = %lld does not cover the %lld visible keys", who,
             (long long)a->num_splits * a->split_span, (long long)decode_visible_max(*a));
  FA_REQUIRE(a->num_splits == 1 || (a->partial_out && a->partial_lse), "%s: splits need partial buffers", who);
  FA_REQUIRE(a->batch <= 65535, "%s: batch exceeds the grid limit", who);
  const int64_t head_groups = decode_head_groups(*a, gt);
  FA_REQUIRE(a->num_splits <= 65535, "%s: too many splits", who);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)head_groups, (unsigned)a->num_splits, (unsigned)a->batch);
  if (gqa.kern) {
    const hipError_t err = hipFuncSetAttribute((const void*)gqa.kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gqa.lds);
    if (err != hipSuccess) {
      fa_set_error("%s: cannot reserve %zu bytes of LDS: %s", who, gqa.lds, hipGetErrorString(err));
      return FA_ERR_LAUNCH;
    }
  }
  hipLaunchKernelGGL(kern, grid, dim3(DEC_THREADS), gqa.kern ? gqa.lds : 0, s, *a, (int)a->split_span);
  int rc = fa_check_launch(who);
  if (rc || a->num_splits == 1) return rc;
  const int64_t rows = partial_rows(*a);
  // Dims per lane: the decode kernels cover Dv <= 256.
  void (*merge)(const fa_attn_args, const int) = a->head_dim_v <= 64    ? decode_merge_kernel<1, 16>
                                               : a->head_dim_v <= 128 ? decode_merge_kernel<2, 16>
                                                                      : decode_merge_kernel<4, 8>;
  hipLaunchKernelGGL(merge, dim3((unsigned)fa_ceil_div(rows, 4)), dim3(256), 0, s, *a, (int)a->split_span);
  return fa_check_launch(who);
}

// Floats of the partial rows; the LSE rows start at the next 256-byte boundary.
int64_t partial_out_floats(const fa_attn_args& a, int64_t splits) {
  return fa_ceil_div(partial_rows(a) * splits * a.head_dim_v, 64) * 64;
}

int64_t partial_floats(const fa_attn_args& a, int64_t splits) {
  return partial_out_floats(a, splits) + partial_rows(a) * splits;
}

// The split plan of the Python host layer (flash_attn_mps_amd/_decode.py
// split_plan with num_splits == 0): spans of 4096 keys halving down to 128
// until the grid holds 1024 workgroups.  Then the split count is reduced
// until the partials fit in `cap_floats` (one split needs no partials).
void plan_splits(const fa_attn_args& a, int gt, int64_t cap_floats, int32_t* splits_out, int32_t* span_out) {
  const int64_t vis = decode_visible_max(a);
  if (vis <= 0) {
    *splits_out = 1;
    *span_out = 32;
    return;
  }
  const int64_t groups = decode_head_groups(a, gt);
  int64_t span = 4096;
  while (span > 128 && a.batch * groups * fa_ceil_div(vis, span) < 1024) span /= 2;
  int64_t splits = fa_ceil_div(vis, span);
  while (splits > 1 && partial_floats(a, splits) > cap_floats) {
    span = fa_ceil_div(fa_ceil_div(vis, fa_ceil_div(splits, 2)), 32) * 32;
    splits = fa_ceil_div(vis, span);
  }
  *splits_out = (int32_t)splits;
  *span_out = (int32_t)(span < INT32_MAX ? span : INT32_MAX);
}

constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[SCRATCH_MAX_DEVICES] = {};

// Device address of this GPU's scratch array: looked up once per device, with
// that device current, and kept.
int scratch_of_device(void* stream, float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SCRATCH_MAX_DEVICES) {
    fa_set_error("fa_decode_fwd_noalloc: no current HIP device");
    return FA_ERR_LAUNCH;
  }
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess || sdev != dev) {
      fa_set_error("fa_decode_fwd_noalloc: the stream does not belong to the current device %d", dev);
      return FA_ERR_INVALID;
    }
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr) {
      fa_set_error("fa_decode_fwd_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(err));
      return FA_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = (float*)p;
  }
  *out = g_scratch_ptr[dev];
  return FA_OK;
}

}  // namespace

extern "C" int fa_decode_fwd(const fa_attn_args* a, void* stream) {
  const int rc = fa_validate_attn(a, "fa_decode_fwd");
  return rc ? rc : decode_launch(a, stream, "fa_decode_fwd");
}

extern "C" int fa_decode_fwd_noalloc(const fa_attn_args* in, void* stream) {
  FA_REQUIRE(in != nullptr, "fa_decode_fwd_noalloc: null args");
  FA_REQUIRE(in->partial_out == nullptr && in->partial_lse == nullptr,
             "fa_decode_fwd_noalloc: partial buffers are library-owned; pass NULL");
  FA_REQUIRE(in->num_splits >= 0, "fa_decode_fwd_noalloc: num_splits must be >= 0");
  fa_attn_args a = *in;
  constexpr int64_t cap = FA_DECODE_SCRATCH_BYTES / (int64_t)sizeof(float);
  if (a.num_splits == 0) {
    FA_REQUIRE(a.batch >= 1 && a.heads_k >= 1 && a.heads_q % a.heads_k == 0,
               "fa_decode_fwd_noalloc: bad batch/head counts");
    int gt = 1;
    if (!pick_decode_gqa(a).kern && !select_decode(a, &gt)) {
      fa_set_error("fa_decode_fwd_noalloc: unsupported dtype/head-dim/stride combination");
      return FA_ERR_UNSUPPORTED;
    }
    plan_splits(a, gt, cap, &a.num_splits, &a.split_span);
  }
  int rc = fa_validate_attn(&a, "fa_decode_fwd_noalloc");
  if (rc) return rc;
  if (a.num_splits > 1) {
    FA_REQUIRE(partial_floats(a, a.num_splits) <= cap,
               "fa_decode_fwd_noalloc: %d splits need %lld bytes of partials; the limit is %lld", a.num_splits,
               (long long)partial_floats(a, a.num_splits) * 4, (long long)FA_DECODE_SCRATCH_BYTES);
    float* base = nullptr;
    rc = scratch_of_device(stream, &base);
    if (rc) return rc;
    a.partial_out = base;
    a.partial_lse = base + partial_out_floats(a, a.num_splits);
  }
  return decode_launch(&a, stream, "fa_decode_fwd_noalloc");
}
