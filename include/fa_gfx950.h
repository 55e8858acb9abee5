/*
 * fa_gfx950.h -- C ABI of libfa_gfx950.so, the MI355X (gfx950) FlashAttention
 * inference kernels behind the flash_attn_mps_amd Python package.
 *
 * Every entry point is extern "C", takes plain device pointers, element
 * strides and sizes, never allocates, never synchronises the host and never
 * reads device memory on the host.  Work is enqueued on the caller's HIP
 * stream (hipStream_t passed as void*).  Each returns 0 on success and a
 * nonzero FA_ERR_* code otherwise; fa_last_error() then describes it.
 *
 * Reference interfaces replaced (paths are inside SuperMarioYL/flash-attn-mps):
 *   fa_store_kvcache   <- _cache.store_kvcache        flash_attn_mps/_cache.py:67-85,
 *                         kernel `store`              flash_attn_mps/kernels/cache.metal:20-39
 *   fa_append_kvcache  <- _cache.append_kvcache       flash_attn_mps/_cache.py:99-127,
 *                         kernel `append`             flash_attn_mps/kernels/cache.metal:41-56
 *   fa_rotary          <- _cache.rotary               flash_attn_mps/_cache.py:130-155,
 *                         kernel `rotate`             flash_attn_mps/kernels/cache.metal:58-76
 *   fa_decode_fwd      <- _decode.decode_attention    flash_attn_mps/_decode.py:40-99,
 *                         kernels `decode_partitions`/`decode_merge`
 *                                                     flash_attn_mps/kernels/attention_decode.metal:18-207
 *   fa_prefill_fwd     <- lib.fast_attention launch   flash_attn_mps/_attention.py:214-221,
 *                         kernel                      flash_attn_mps/kernels/attention_fast.metal:103-597
 *   fa_attn_fwd        <- attention_tiled/attention_vector launch
 *                                                     flash_attn_mps/_attention.py:222-237,
 *                                                     flash_attn_mps/kernels/attention.metal:60-248
 *   fa_merge_partials  <- _merge._merge_partials      flash_attn_mps/_merge.py:44-57,
 *                         kernel `merge_partials`     flash_attn_mps/kernels/merge.metal:30-58
 *   fa_merge_pair      <- _merge.merge_attn_states    flash_attn_mps/_merge.py:20-41,
 *                         kernel `merge_pair`         flash_attn_mps/kernels/merge.metal:9-28
 * The reference binds its kernels through torch.mps.compile_shader(...).<kernel>(
 * tensors..., int64 params, float params, threads=, group_size=); the structs
 * below carry the same information (the `_META` vectors of
 * flash_attn_mps/_attention.py:10-16 and flash_attn_mps/_decode.py:7-8).
 */
#ifndef FA_GFX950_H
#define FA_GFX950_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 3: fa_decode_fwd's split partials became split-major ([batch, S, R, Hq,
 * Dv]; the struct layouts are those of version 2). */
#define FA_ABI_VERSION 3

/* Element types of attention/cache tensors. */
enum fa_dtype { FA_F16 = 0, FA_BF16 = 1, FA_F32 = 2, FA_E4M3 = 3 };
/* Integer types of slot mappings. */
enum fa_index_dtype { FA_I32 = 0, FA_I64 = 1 };

/* Return codes. */
enum fa_status {
  FA_OK = 0,
  FA_ERR_INVALID = 1,     /* inconsistent arguments (null pointer, bad shape) */
  FA_ERR_UNSUPPORTED = 2, /* combination not compiled into this entry point */
  FA_ERR_LAUNCH = 3       /* hipLaunchKernel / hipGetLastError failure */
};

/* ---------------------------------------------------------------- caches */

/* One tensor/cache pair of store_kvcache: cache[slot / P, slot % P, h, d] = x[t, h, d].
 * Slots < 0 or >= num_pages * page_size are skipped.  When cache_dtype is
 * FA_E4M3 the value stored is E4M3FN(x / scale[h * scale_stride]) with RNE,
 * saturation to +-448 and NaN -> sign|0x7F; otherwise the bits are copied. */
typedef struct fa_store_desc {
  const void* x;           /* [tokens, heads, dim] */
  void* cache;             /* [num_pages, page_size, heads, dim] */
  const float* scale;      /* [1] or [heads]; only read for FA_E4M3 caches */
  int32_t x_dtype;         /* FA_F16 / FA_BF16 / FA_F32 */
  int32_t cache_dtype;     /* x_dtype or FA_E4M3 */
  int64_t heads, dim;
  int64_t x_stride[3];
  int64_t cache_stride[4];
  int64_t scale_stride;    /* 0: one scale, 1: per head */
} fa_store_desc;

typedef struct fa_store_args {
  fa_store_desc kv[2];     /* K and V; kv[1].x == NULL stores only kv[0] */
  const void* slots;       /* [tokens] int32 or int64 */
  int32_t slot_dtype;      /* FA_I32 / FA_I64 */
  int32_t _pad0;
  int64_t slot_stride;
  int64_t tokens;
  int64_t page_size;
  int64_t num_pages;
} fa_store_args;

/* One tensor/cache pair of append_kvcache: x[b, j] goes to position
 * lengths[b] + j of cache row (batch_index ? batch_index[b] : b), either
 * directly (dense cache) or through block_table[row, pos / P] (paged).  Out of
 * range rows, positions or blocks are skipped. */
typedef struct fa_append_args {
  fa_store_desc kv[2];     /* x is [batch, new_tokens, heads, dim]; x_stride[0..2] are
                              the (new_token, head, dim) strides, batch stride below */
  int64_t x_batch_stride[2];
  const int32_t* lengths;      /* [batch] int32 contiguous */
  const int32_t* batch_index;  /* [batch] int32 contiguous, or NULL */
  const int32_t* block_table;  /* [rows, cols] int32 contiguous, or NULL */
  int64_t batch, new_tokens;
  int64_t page_size;           /* cache.shape[1] (capacity when dense) */
  int64_t num_blocks;          /* cache.shape[0] */
  int64_t table_rows, table_cols;
} fa_append_args;

/* Rotary position embedding of [batch, seq, heads, dim] into a contiguous
 * output; positions lengths[b] + (advance ? j : 0); cos/sin [positions, rot/2]
 * fp32 contiguous. */
typedef struct fa_rotary_args {
  const void* x; void* out;
  const float* cos_table; const float* sin_table;
  const int32_t* lengths;
  int32_t dtype;           /* FA_F16 / FA_BF16 / FA_F32 */
  int32_t interleaved;
  int32_t advance;
  int32_t _pad0;
  int64_t batch, seq, heads, dim, half_rot, table_rows;
  int64_t x_stride[4];
} fa_rotary_args;

/* ------------------------------------------------------------- attention */

/* Attention over packed [T, Hkv, D] or paged [pages, P, Hkv, D] K/V.  Output
 * [total_q, Hq, Dv] and natural-log LSE [Hq, total_q].  All strides are in
 * elements.  Optional pointers are NULL when absent. */
typedef struct fa_attn_args {
  const void* q; const void* k; const void* v;
  void* out;
  float* lse;
  int32_t q_dtype, k_dtype, v_dtype, out_dtype;

  int64_t total_q, heads_q, heads_k, head_dim_qk, head_dim_v, batch;
  int64_t page_size;                 /* 0: packed 3-D K/V */
  int64_t max_seqlen_q, max_seqlen_k;

  int64_t q_stride[3], k_stride[4], v_stride[4], out_stride[3], lse_stride[2];

  const int32_t* cu_seqlens_q; int64_t cu_q_stride;
  const int32_t* cu_seqlens_k; int64_t cu_k_stride;
  const int32_t* seqused_k;    int64_t used_k_stride;
  const int32_t* block_table;  int64_t bt_stride[2];
  const int32_t* leftpad_k;    int64_t leftpad_stride;

  int32_t causal;                    /* static lower-right causal flag */
  int32_t window_left, window_right; /* -1: unbounded */
  int32_t mask_kind;                 /* 0 none, 1 mm-prefix ranges, 2 rolling window + prefix */
  int32_t mask_window, mask_clamp;
  const uint8_t* causal_by_batch; int64_t causal_stride;   /* dynamic causal bool [B] */
  const int32_t* mask_ranges;     int64_t ranges_stride[2]; /* kind 1: [T, 2] */
  const int32_t* mask_prefix;     int64_t prefix_stride;    /* kind 2: [B] */
  const int32_t* mask_window_len;                           /* kind 2: [1] */

  float softmax_scale, softcap;      /* softcap 0: disabled */
  const float* alibi;     int64_t alibi_stride[2];  /* [B, Hq] or [Hq] (stride[0] = 0) */
  const float* sinks;     int64_t sink_stride;      /* [Hq] fp32 */
  const float* q_descale; int64_t q_descale_stride[2]; /* [B, Hkv] */
  const float* k_descale; int64_t k_descale_stride[2];
  const float* v_descale; int64_t v_descale_stride[2];

  int32_t num_splits;                /* >= 1 */
  int32_t split_span;                /* fa_decode_fwd: keys per split (>= 1); the splits
                                        must cover every visible key:
                                        num_splits * split_span >= min(max_seqlen_k,
                                        window_left + R) (window_left < 0: max_seqlen_k),
                                        R = max(1, max_seqlen_q) */
  float* partial_out;                /* num_splits > 1: caller-owned fp32 workspace,
                                        fa_decode_fwd [batch, S, R, Hq, Dv] contiguous,
                                        fa_attn_fwd [S, total_q, Hq, Dv] contiguous */
  float* partial_lse;                /* fa_decode_fwd [batch, R, Hq, S], fa_attn_fwd [S, Hq, total_q] */

  int32_t flags;                     /* FA_FLAG_* bits */
  int32_t _pad1;
} fa_attn_args;

/* fa_attn_args.flags: fa_prefill_fwd leaves requests with exactly one query
 * row untouched (a caller routes those to fa_decode_fwd in the same batch). */
#define FA_FLAG_SKIP_SINGLE_QUERY 1

/* Two-state merge (out may alias a or b, out_lse may alias a_lse). */
typedef struct fa_merge_pair_args {
  void* out; const void* a; const void* b;
  const float* a_lse; const float* b_lse; float* out_lse;  /* out_lse may be NULL */
  int32_t dtype; int32_t _pad0;
  int64_t tokens, heads, dim;
  int64_t out_stride[3], a_stride[3], b_stride[3];
  int64_t a_lse_stride[2], b_lse_stride[2], out_lse_stride[2];
} fa_merge_pair_args;

/* N-way merge of partial states [S, T, H, D] (any dtype) / [S, H, T] fp32 into
 * out [T, H, D] and lse [H, T] (both with strides). */
typedef struct fa_merge_partials_args {
  const void* partial; const float* partial_lse;
  void* out; float* lse;
  int32_t partial_dtype, out_dtype;
  int64_t splits, tokens, heads, dim;
  int64_t partial_stride[4], partial_lse_stride[3];
  int64_t out_stride[3], lse_stride[2];
} fa_merge_partials_args;

/* ----------------------------------------------------------- entry points */

int fa_abi_version(void);
/* sizeof() of each argument struct, for binding checks:
 * [store, append, rotary, attn, merge_pair, merge_partials]. */
void fa_struct_sizes(int64_t* sizes6);
const char* fa_last_error(void);

int fa_store_kvcache(const fa_store_args* args, void* stream);
int fa_append_kvcache(const fa_append_args* args, void* stream);
int fa_rotary(const fa_rotary_args* args, void* stream);

/* Split-KV decode.  With max_seqlen_q <= 1: one query row per request (rows
 * with cu_seqlens_q difference 1; others are skipped).  With max_seqlen_q = R
 * in 2..16 (speculative / multi-token decode; no counterpart in the
 * reference, which runs such rows through its prefill kernel): requests of
 * 1..R rows, the rows being the request's last key positions (causal and
 * windows bottom-right aligned), on the matrix-core kernel only --
 * fa_decode_supported says whether it takes the arguments.  Writes out/lse
 * directly when num_splits == 1, otherwise fills partial_out
 * [batch, S, R, Hq, Dv] / partial_lse [batch, R, Hq, S] (R = 1 for one row)
 * and merges. */
int fa_decode_supported(const fa_attn_args* args);
int fa_decode_fwd(const fa_attn_args* args, void* stream);

/* fa_decode_fwd that allocates nothing.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc).  The split
 * partials live in a library-owned device array of FA_DECODE_SCRATCH_BYTES
 * per GPU, held until the process ends; args->partial_out/partial_lse must
 * be NULL.  num_splits == 0 lets the library plan the splits (spans start at
 * 2048 keys and halve down to 128 until the grid holds at least 2048
 * workgroups -- the plan of the Python host layer -- then the split count is
 * reduced until the partials fit; one split needs none); otherwise the
 * caller's num_splits/split_span are used and
 * batch * R * Hq * num_splits * (Dv + 1) * 4 bytes must fit, else FA_ERR_INVALID.
 * Every call on one GPU shares that GPU's array and the array keeps the last
 * call's partials (nothing in it needs clearing: each split writes its own
 * rows before the merge reads them); calls that overlap in time on one GPU
 * (two streams, two threads) race.  The stream must belong to the current
 * device. */
#define FA_DECODE_SCRATCH_BYTES (32ll << 20)
int fa_decode_fwd_noalloc(const fa_attn_args* args, void* stream);

/* MFMA prefill (bf16/fp16 queries over bf16/fp16 or FP8 E4M3 K/V with
 * descales, or E4M3 queries over E4M3 K/V; causal, per-request causal,
 * windows, softcap, sinks, vLLM mask kinds 1 and 2, and ALiBi, which
 * combines with softcap, windows, per-request causality and E4M3 K/V at
 * unpadded 64/128/256-dim heads; head dims 32-256 and 192/128).
 * fa_prefill_supported() says whether the argument
 * combination is compiled in.  With FA_FLAG_SKIP_SINGLE_QUERY in
 * args->flags, requests with one query row are left untouched for
 * fa_decode_fwd (no reference counterpart: the reference runs such rows
 * through its prefill tile, flash_attn_mps/_attention.py:149-158). */
int fa_prefill_supported(const fa_attn_args* args);
int fa_prefill_fwd(const fa_attn_args* args, void* stream);

/* Generic fused attention: every feature, dims 1..512, any strides and
 * dtypes.  num_splits > 1 requires partial_out [S, T, Hq, Dv] and
 * partial_lse [S, Hq, T] and merges into out/lse. */
int fa_attn_fwd(const fa_attn_args* args, void* stream);

int fa_merge_pair(const fa_merge_pair_args* args, void* stream);
int fa_merge_partials(const fa_merge_partials_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FA_GFX950_H */
