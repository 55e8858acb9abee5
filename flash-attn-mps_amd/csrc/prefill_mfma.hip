// Host side of the MFMA prefill: kernel selection, the support predicate and
// the C-ABI entry points fa_prefill_supported / fa_prefill_fwd (replacing
// the reference's `fast_attention` dispatch, flash_attn_mps/_attention.py:
// 149-158, 170-238).  The kernel itself is in prefill_kernel.h; its variants
// are instantiated in prefill_inst_*.hip.
#include "prefill_kernel.h"

namespace {

using namespace fa_prefill;

// Windows, or per-request causality (run as a right window of 0 per request).
bool window_set(const fa_attn_args& a) {
  return a.window_left >= 0 || a.causal_by_batch || (a.causal == 0 && a.window_right >= 0);
}

PrefillChoice select_prefill(const fa_attn_args& a) {
  const bool causal = a.causal != 0, fp8 = a.k_dtype == FA_E4M3;
  // plain / softcap / ALiBi / softcap then ALiBi
  const int score = a.alibi ? (a.softcap > 0.0f ? 3 : 2) : a.softcap > 0.0f ? 1 : 0;
  // vLLM mask kinds carry their own causality and windows (the causal and
  // window fields do not apply to them, kernels/attention.metal:29-45).
  const int mk = a.mask_kind;
  // A right window bounds nothing under causality.
  const bool win = mk == 0 && window_set(a);
  const int64_t dq = a.head_dim_qk, dv = a.head_dim_v;
  if (a.q_dtype == FA_E4M3) return pick_fp8q(a.out_dtype, dq, dv, causal, score, win);
  const bool bf16 = a.q_dtype == FA_BF16;
  if (!fp8 && dq <= 128)
    return bf16 ? pick_bf16_small(dq, dv, causal, score, win, mk) : pick_f16_small(dq, dv, causal, score, win, mk);
  return bf16 ? pick_bf16_large(dq, dv, causal, score, win, fp8, mk)
              : pick_f16_large(dq, dv, causal, score, win, fp8, mk);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool prefill_ok(const fa_attn_args& a) {
  const bool fp8 = a.k_dtype == FA_E4M3, fp8q = a.q_dtype == FA_E4M3;
  const int64_t dq = a.head_dim_qk, dv = a.head_dim_v;
  if (a.k_dtype != a.v_dtype) return false;
  if (fp8q) {
    // E4M3 queries: E4M3 K/V, 16-bit output.
    if (!fp8 || (a.out_dtype != FA_F16 && a.out_dtype != FA_BF16)) return false;
  } else {
    if (a.q_dtype != FA_BF16 && a.q_dtype != FA_F16) return false;
    if (a.out_dtype != a.q_dtype) return false;
    if (!fp8 && a.k_dtype != a.q_dtype) return false;
  }
  if (fp8) {
    if (!(dq == dv && (dq == 64 || dq == 128 || dq == 256))) return false;
  } else if (!((dq == dv && (dq == 32 || dq == 64 || dq == 72 || dq == 80 || dq == 96 || dq == 128 || dq == 256)) ||
               (dq == 192 && dv == 128))) {
    return false;
  }
  // Left padding shifts a request's storage positions; a 16-key group must
  // then still lie in one page: packed K/V, or one page per request (the
  // dense-cache layout of flash_attn_with_kvcache).
  if (a.leftpad_k && a.page_size && a.max_seqlen_k > a.page_size) return false;
  if (a.mask_kind != 0) {
    // vLLM mask kinds 1 / 2 (vllm.mm_prefix_mask / rswa_mask) on unpadded
    // head dims, 16-bit queries, without ALiBi; key ranges use +-2^29
    // sentinels, so keys stay below 2^28.
    if (a.mask_kind != 1 && a.mask_kind != 2) return false;
    if (fp8q || a.alibi || a.max_seqlen_k >= (1ll << 28)) return false;
    if (a.mask_kind == 1 && !a.mask_ranges) return false;
    if (a.mask_kind == 2 && (!a.mask_prefix || !a.mask_window_len)) return false;
    if (!((dq == dv && (dq == 64 || dq == 128 || dq == 256)) || (dq == 192 && dv == 128))) return false;
  }
  // ALiBi (per-head or per-request slopes): any 16-bit head dim alone; with
  // softcap, windows, per-request causality or E4M3 K/V, unpadded 64 / 128 /
  // 256-dim heads; not with E4M3 queries.
  if (a.alibi) {
    if (fp8q) return false;
    if ((a.softcap > 0.0f || window_set(a) || fp8) && !(dq == dv && (dq == 64 || dq == 128 || dq == 256)))
      return false;
  }
  const int kb = fp8 ? 1 : 2;   // K/V bytes per element
  if (a.window_left < -1 || a.window_right < -1) return false;
  if (a.num_splits != 1) return false;
  if (a.q_stride[2] != 1 || a.k_stride[3] != 1 || a.v_stride[3] != 1 || a.out_stride[2] != 1) return false;
  if (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.v) || ((uintptr_t)a.out & 7u)) return false;
  const int qb = fp8q ? 1 : 2;   // query bytes per element
  for (int i = 0; i < 2; ++i)
    if ((a.q_stride[i] * qb) % 16 || (a.out_stride[i] * 2) % 8) return false;
  for (int i = a.page_size ? 0 : 1; i < 3; ++i)
    if ((a.k_stride[i] * kb) % 16 || (a.v_stride[i] * kb) % 16) return false;
  // Group-bounded buffer loads need non-overlapping rows and 16-row groups
  // that span less than 2 GiB.
  if (a.k_stride[1] < dq || a.v_stride[1] < dv) return false;
  if (16 * a.k_stride[1] * kb >= 0x7fffffffll || 16 * a.v_stride[1] * kb >= 0x7fffffffll) return false;
  if (a.page_size) {
    // Power-of-two pages (the kernel splits a position into page and slot
    // with a shift and a mask), or one page holding every key: a dense cache
    // [B, capacity, Hkv, D] seen through a one-column table, whose positions
    // stay below max_seqlen_k <= capacity < 2^log2_page, so the page index
    // is always 0 whatever the capacity.
    if (a.page_size < 16 || ((a.page_size & (a.page_size - 1)) && a.max_seqlen_k > a.page_size)) return false;
    // Page strides are 32-bit byte counts in the group descriptors.
    if (kb * a.k_stride[0] >= (1ll << 32) || kb * a.v_stride[0] >= (1ll << 32)) return false;
  }
  return true;
}

}  // namespace

extern "C" int fa_prefill_supported(const fa_attn_args* a) {
  return a != nullptr && prefill_ok(*a);
}

extern "C" int fa_prefill_fwd(const fa_attn_args* a, void* stream) {
  int rc = fa_validate_attn(a, "fa_prefill_fwd");
  if (rc) return rc;
  if (!prefill_ok(*a)) {
    fa_set_error("fa_prefill_fwd: combination not supported by the MFMA kernel");
    return FA_ERR_UNSUPPORTED;
  }
  if (a->total_q == 0) return FA_OK;
  FA_REQUIRE(a->max_seqlen_q >= 1, "fa_prefill_fwd: max_seqlen_q must be positive");
  PrefillChoice ch = select_prefill(*a);
  FA_REQUIRE(ch.kern != nullptr && ch.vparts >= 1, "fa_prefill_fwd: no kernel instance for these arguments");
  PrefillShape shp;
  // Query heads per workgroup: two heads of a KV head share each workgroup's
  // K/V tiles when the GQA group is even.
  shp.hp = (a->heads_q / a->heads_k) % 2 == 0 ? 2 : 1;
  const int64_t bmh = ch.bm / shp.hp;   // query rows per head of a workgroup
  shp.n_qblocks = (int)fa_ceil_div(a->max_seqlen_q, bmh);
  shp.log2_page = 0;
  if (a->page_size)
    while ((1ll << shp.log2_page) < a->page_size) ++shp.log2_page;
  const int64_t pairs = a->batch * a->heads_k;
  const int64_t group = a->heads_q / a->heads_k / shp.hp;   // workgroups per query block and KV head
  int64_t blocks = fa_ceil_div(pairs, 8) * 8 * shp.n_qblocks * group;
  // Compact work list: requests hold at most sum ceil(q_len / bmh) <=
  // (T + B (bmh - 1)) / bmh query blocks per KV head; an XCD owns Hkv / g KV
  // heads (g = gcd(Hkv, 8)) and every S-th block of each (S = 8 / g): at most
  // sum ceil(n_b / S) <= (qblocks + B (S - 1)) / S blocks per head.
  shp.compact = 0;
  if (a->batch <= PF_COMPACT_MAX_BATCH) {
    const int64_t qblocks = (a->total_q + a->batch * (bmh - 1)) / bmh;
    const int64_t hk = a->heads_k, gk = hk % 8 == 0 ? 8 : hk % 4 == 0 ? 4 : hk % 2 == 0 ? 2 : 1;
    const int64_t S = 8 / gk;
    const int64_t per_xcd = (hk / gk) * ((qblocks + a->batch * (S - 1)) / S);
    const int64_t compact = 8 * group * per_xcd;
    if (compact < blocks) {
      blocks = compact;
      shp.compact = 1;
    }
  }
  // V column parts: each work item runs as vparts workgroups (blocks is a
  // multiple of 8, as the kernel's 16-block interleave of the parts needs).
  blocks *= ch.vparts;
  FA_REQUIRE(blocks <= 0x7fffffffll, "fa_prefill_fwd: grid too large");
  hipError_t err = hipFuncSetAttribute((const void*)ch.kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)ch.lds);
  if (err != hipSuccess) {
    fa_set_error("fa_prefill_fwd: cannot reserve %zu bytes of LDS: %s", ch.lds, hipGetErrorString(err));
    return FA_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(ch.kern, dim3((unsigned)blocks), dim3(ch.threads), ch.lds, (hipStream_t)stream, *a, shp);
  return fa_check_launch("fa_prefill_fwd");
}
