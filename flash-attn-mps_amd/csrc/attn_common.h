// Per-request metadata and masking rules shared by the attention kernels.
//
// Semantics follow flash_attn_mps/kernels/attention.metal:18-51 and
// flash_attn_mps/tests/reference.py:38-90: lower-right causality (query row i
// of a request with Lq queries and Lk keys sits at absolute position
// i + Lk - Lq), windows measured on those absolute positions, the score
// transform scale*dot -> softcap -> minus ALiBi, and the two vLLM mask kinds.
#pragma once

#include "fa_device.h"

struct RequestInfo {
  int q_begin, q_len;   // packed query rows of this request
  int k_len;            // visible keys (seqused_k or cu_k difference)
  int k_base;           // packed K/V row of key 0 (0 when paged)
  int left;             // left padding added to storage positions
  bool causal;
};

// The metadata is read-only for the whole launch, so it is read through the
// scalar cache (uniform values stay in SGPRs for every caller with a uniform b).
FA_DEV RequestInfo load_request(const fa_attn_args& a, int64_t b) {
  RequestInfo r;
  r.q_begin = load_invariant_i32(a.cu_seqlens_q, b * a.cu_q_stride);
  r.q_len = load_invariant_i32(a.cu_seqlens_q, (b + 1) * a.cu_q_stride) - r.q_begin;
  const int kcu = a.cu_seqlens_k ? load_invariant_i32(a.cu_seqlens_k, b * a.cu_k_stride) : 0;
  r.k_base = a.page_size ? 0 : kcu;
  r.k_len = a.seqused_k ? load_invariant_i32(a.seqused_k, b * a.used_k_stride)
                        : load_invariant_i32(a.cu_seqlens_k, (b + 1) * a.cu_k_stride) - kcu;
  r.left = a.leftpad_k ? load_invariant_i32(a.leftpad_k, b * a.leftpad_stride) : 0;
  r.causal = a.causal_by_batch ? a.causal_by_batch[b * a.causal_stride] != 0 : a.causal != 0;
  return r;
}

// Element offset of key/value `token` (0-based within the request) of KV head kh.
FA_DEV int64_t kv_offset(const fa_attn_args& a, const int64_t* st, int64_t b,
                         const RequestInfo& r, int token, int kh) {
  const int64_t pos = (int64_t)r.k_base + r.left + token;
  if (a.page_size) {
    const int64_t page = pos / a.page_size;
    const int64_t blk = a.block_table[b * a.bt_stride[0] + page * a.bt_stride[1]];
    return blk * st[0] + (pos - page * a.page_size) * st[1] + (int64_t)kh * st[2];
  }
  return pos * st[1] + (int64_t)kh * st[2];
}

// Whether key `token` is visible from the query at absolute position q_abs
// (packed query row tq).
FA_DEV bool key_allowed(const fa_attn_args& a, int64_t b, int token, int q_abs, int64_t tq, bool causal) {
  const int diff = q_abs - token;
  if (a.mask_kind == 1) {
    const bool local = diff >= 0 && (a.mask_window < 0 || diff < a.mask_window);
    const int lo = a.mask_ranges[tq * a.ranges_stride[0]];
    const int hi = a.mask_ranges[tq * a.ranges_stride[0] + a.ranges_stride[1]];
    bool modality = lo >= 0 && token >= lo && token <= hi;
    if (a.mask_clamp) modality = modality && (a.mask_window < 0 || diff < a.mask_window);
    return local || modality;
  }
  if (a.mask_kind == 2)
    return diff >= 0 && (token < a.mask_prefix[b * a.prefix_stride] || diff < a.mask_window_len[0]);
  return (!causal || diff >= 0) && (a.window_left < 0 || diff <= a.window_left) &&
         (a.window_right < 0 || -diff <= a.window_right);
}

FA_DEV float descale_of(const float* p, const int64_t* st, int64_t b, int kh) {
  return p ? p[b * st[0] + (int64_t)kh * st[1]] : 1.0f;
}

// Host-side argument checks shared by fa_attn_fwd / fa_decode_fwd / fa_prefill_fwd.
int fa_validate_attn(const fa_attn_args* a, const char* who);
