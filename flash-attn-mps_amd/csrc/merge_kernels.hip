// Log-sum-exp merges of independently computed attention states.
//
// merge_pair restates flash_attn_mps/kernels/merge.metal:9-28 and
// merge_partials merge.metal:30-58: weights w_s = exp(lse_s - max) (an LSE of
// +inf takes all the weight, equally shared among +inf states), states with
// zero weight are never read (so NaN payloads of empty states vanish), an
// all -inf row gives output 0 and LSE -inf.  One wave owns a (token, head)
// row: its lanes take the head dimension 64 elements at a time (consecutive
// elements in consecutive lanes, so each load and store instruction is one
// contiguous segment of the row), and every lane computes the row's weights.
// In-place merging (out or out_lse aliasing an input) is safe: each element
// is read and written by the same lane, and the LSE inputs are read by the
// whole wave before lane 0 writes the merged LSE.
#include "fa_device.h"

namespace {

FA_DEV float merge_weight(float l, float peak) {
  if (peak == -INFINITY) return 0.0f;
  if (peak == INFINITY) return l == peak ? 1.0f : 0.0f;
  return expf(l - peak);
}

struct MergePairParams {
  void* out;
  const void* a;
  const void* b;
  const float* al;
  const float* bl;
  float* ol;
  int64_t tokens, heads, dim;
  int64_t os[3], as[3], bs[3], als[2], bls[2], ols[2];
};

template <typename T>
__global__ __launch_bounds__(256) void merge_pair_kernel(const MergePairParams p) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= p.tokens * p.heads) return;
  const int64_t t = row / p.heads, h = row - t * p.heads;
  const float la = p.al[h * p.als[0] + t * p.als[1]];
  const float lb = p.bl[h * p.bls[0] + t * p.bls[1]];
  const float peak = fmaxf(la, lb);
  const bool empty = peak == -INFINITY;
  const float wa = merge_weight(la, peak), wb = merge_weight(lb, peak);
  const float total = wa + wb;
  for (int64_t d = lane; d < p.dim; d += 64) {
    float v = 0.0f;
    if (wa > 0.0f) v += wa * load_elem<T>(p.a, t * p.as[0] + h * p.as[1] + d * p.as[2]);
    if (wb > 0.0f) v += wb * load_elem<T>(p.b, t * p.bs[0] + h * p.bs[1] + d * p.bs[2]);
    if (!empty) v /= total;
    store_elem<T>(p.out, t * p.os[0] + h * p.os[1] + d * p.os[2], v);
  }
  if (p.ol && lane == 0) p.ol[h * p.ols[0] + t * p.ols[1]] = empty ? -INFINITY : peak + logf(total);
}

struct MergePartialsParams {
  const void* part;
  const float* plse;
  void* out;
  float* lse;
  int64_t splits, tokens, heads, dim;
  int64_t ps[4], pls[3], os[3], ls[2];
  int32_t part_dtype, out_dtype;
};

__global__ __launch_bounds__(256) void merge_partials_kernel(const MergePartialsParams p) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= p.tokens * p.heads) return;
  const int64_t t = row / p.heads, h = row - t * p.heads;
  float peak = -INFINITY;
  for (int64_t s = 0; s < p.splits; ++s) peak = fmaxf(peak, p.plse[s * p.pls[0] + h * p.pls[1] + t * p.pls[2]]);
  const bool empty = peak == -INFINITY;
  float denom = 0.0f;
  for (int64_t s = 0; s < p.splits; ++s) denom += merge_weight(p.plse[s * p.pls[0] + h * p.pls[1] + t * p.pls[2]], peak);
  for (int64_t d = lane; d < p.dim; d += 64) {
    float v = 0.0f;
    if (!empty) {
      for (int64_t s = 0; s < p.splits; ++s) {
        const float w = merge_weight(p.plse[s * p.pls[0] + h * p.pls[1] + t * p.pls[2]], peak);
        if (w > 0.0f) v += w * load_any(p.part, s * p.ps[0] + t * p.ps[1] + h * p.ps[2] + d * p.ps[3], p.part_dtype);
      }
      v /= denom;
    }
    store_any(p.out, t * p.os[0] + h * p.os[1] + d * p.os[2], p.out_dtype, v);
  }
  if (lane == 0) p.lse[h * p.ls[0] + t * p.ls[1]] = empty ? -INFINITY : peak + logf(denom);
}

}  // namespace

extern "C" int fa_merge_pair(const fa_merge_pair_args* a, void* stream) {
  FA_REQUIRE(a && a->out && a->a && a->b && a->a_lse && a->b_lse, "fa_merge_pair: null argument");
  FA_REQUIRE(a->dtype == FA_F16 || a->dtype == FA_BF16 || a->dtype == FA_F32, "fa_merge_pair: dtype must be f16/bf16/f32");
  MergePairParams p;
  p.out = a->out; p.a = a->a; p.b = a->b;
  p.al = a->a_lse; p.bl = a->b_lse; p.ol = a->out_lse;
  p.tokens = a->tokens; p.heads = a->heads; p.dim = a->dim;
  for (int i = 0; i < 3; ++i) { p.os[i] = a->out_stride[i]; p.as[i] = a->a_stride[i]; p.bs[i] = a->b_stride[i]; }
  for (int i = 0; i < 2; ++i) { p.als[i] = a->a_lse_stride[i]; p.bls[i] = a->b_lse_stride[i]; p.ols[i] = a->out_lse_stride[i]; }
  const int64_t rows = p.tokens * p.heads;
  if (rows == 0) return FA_OK;
  FA_REQUIRE(fa_ceil_div(rows, 4) <= 0x7fffffffll, "fa_merge_pair: too many rows");
  const dim3 grid((unsigned)fa_ceil_div(rows, 4));   // a wave per row
  hipStream_t s = (hipStream_t)stream;
  switch (a->dtype) {
    case FA_F16: hipLaunchKernelGGL(merge_pair_kernel<F16T>, grid, dim3(256), 0, s, p); break;
    case FA_BF16: hipLaunchKernelGGL(merge_pair_kernel<BF16T>, grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(merge_pair_kernel<F32T>, grid, dim3(256), 0, s, p); break;
  }
  return fa_check_launch("fa_merge_pair");
}

extern "C" int fa_merge_partials(const fa_merge_partials_args* a, void* stream) {
  FA_REQUIRE(a && a->out && a->lse && (a->splits == 0 || (a->partial && a->partial_lse)),
             "fa_merge_partials: null argument");
  FA_REQUIRE(a->out_dtype == FA_F16 || a->out_dtype == FA_BF16 || a->out_dtype == FA_F32,
             "fa_merge_partials: output dtype must be f16/bf16/f32");
  FA_REQUIRE(a->partial_dtype == FA_F16 || a->partial_dtype == FA_BF16 || a->partial_dtype == FA_F32,
             "fa_merge_partials: partial dtype must be f16/bf16/f32");
  MergePartialsParams p;
  p.part = a->partial; p.plse = a->partial_lse; p.out = a->out; p.lse = a->lse;
  p.splits = a->splits; p.tokens = a->tokens; p.heads = a->heads; p.dim = a->dim;
  for (int i = 0; i < 4; ++i) p.ps[i] = a->partial_stride[i];
  for (int i = 0; i < 3; ++i) { p.pls[i] = a->partial_lse_stride[i]; p.os[i] = a->out_stride[i]; }
  for (int i = 0; i < 2; ++i) p.ls[i] = a->lse_stride[i];
  p.part_dtype = a->partial_dtype; p.out_dtype = a->out_dtype;
  const int64_t rows = p.tokens * p.heads;
  if (rows == 0) return FA_OK;
  FA_REQUIRE(fa_ceil_div(rows, 4) <= 0x7fffffffll, "fa_merge_partials: too many rows");
  hipLaunchKernelGGL(merge_partials_kernel, dim3((unsigned)fa_ceil_div(rows, 4)), dim3(256), 0,   // a wave per row
                     (hipStream_t)stream, p);
  return fa_check_launch("fa_merge_partials");
}
