// Variants of the matrix-core GQA decode kernel (decode_gqa.h) and their
// selection: 16-bit queries over K/V of the same type or E4M3, Dqk = Dv in
// {64, 128}, with and without softcap; neighbouring 64-dim heads, and
// 128-dim E4M3 heads, stored next to each other run two KV heads per
// workgroup (PACK = 2).
#include "decode_gqa.h"

namespace fa_decode {

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Every 16-byte chunk the kernel loads starts on a 16-byte boundary: row,
// head and page strides of K/V (`kvb` bytes per element) and the query's
// token and head strides.
bool chunks_aligned(const fa_attn_args& a, int kvb) {
  if (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.v)) return false;
  if (a.q_stride[2] != 1 || a.k_stride[3] != 1 || a.v_stride[3] != 1) return false;
  for (int i = 0; i < 2; ++i)
    if ((a.q_stride[i] * 2) % 16) return false;
  for (int i = 0; i < 3; ++i)
    if ((a.k_stride[i] * kvb) % 16 || (a.v_stride[i] * kvb) % 16 || a.k_stride[i] < 0 || a.v_stride[i] < 0)
      return false;
  return true;
}

template <typename T, typename KT, int D, int PACK>
GqaChoice choose(bool cap) {
  GqaChoice c;
  c.kern = cap ? fa_decode_gqa::decode_gqa_kernel<T, D, true, KT, PACK>
               : fa_decode_gqa::decode_gqa_kernel<T, D, false, KT, PACK>;
  c.lds = fa_decode_gqa::gqa_lds_bytes<D, KT::id == FA_E4M3, PACK>();
  c.pack = PACK;
  return c;
}

// Two KV heads per workgroup (64-dim heads, or 128-dim E4M3 heads) when
// every key row holds them next to each other (head stride = the head dim,
// rows of two heads or more), both heads' query columns fit one 32-column
// tile (a second tile would read both heads' rows again: 48/2 heads at 16
// bits 4.82 -> 2.64 TB/s), and the cache is E4M3 or has 8 KV heads or more.
// Measured in one process against the unpaired kernel on the same caches,
// calls alternated (64 requests of U[512, 32768] keys, one query row): E4M3
// d64 32/8 2.94 -> 5.18 TB/s, 16/8 2.97 -> 5.25 (64-byte rows are the worst
// case of the paged gather); 16-bit d64 32/8 5.32 -> 5.68, 16/16 5.74 ->
// 6.07; E4M3 d128 32/8 5.39 -> 5.70, 64/8 5.06 -> 5.37, 12/4 4.91 -> 4.88.
// With few KV heads 16-bit pairing loses (separate processes: 12/4 5.58 ->
// 5.33, 14/2 5.01 -> 4.74): a key row is then 256-512 bytes that the heads'
// workgroups already read side by side, and pairing halves the workgroups.
// Paired 64-dim heads also take groups of 1 and 2, which otherwise run on
// the VALU kernel (separate processes: E4M3 16/16 3.06 -> 5.64, 16/8 2.91
// -> 4.92; 16-bit 16/16 5.94 -> 6.29, 16/8 the same).
bool packable(const fa_attn_args& a) {
  const int64_t ntok = a.max_seqlen_q > 1 ? a.max_seqlen_q : 1, d = a.head_dim_qk;
  const bool fp8 = a.k_dtype == FA_E4M3;
  if (!(d == 64 || (d == 128 && fp8))) return false;
  return a.heads_k % 2 == 0 && a.k_stride[2] == d && a.v_stride[2] == d && a.k_stride[1] >= 2 * d &&
         a.v_stride[1] >= 2 * d && 2 * (a.heads_q / a.heads_k) * ntok <= fa_decode_gqa::GQA_HEADS &&
         (fp8 || a.heads_k >= 8);
}

template <typename T, typename KT>
GqaChoice choose_dim(const fa_attn_args& a, bool cap) {
  if (a.head_dim_qk == 64) return packable(a) ? choose<T, KT, 128, 2>(cap) : choose<T, KT, 64, 1>(cap);
  if constexpr (KT::id == FA_E4M3) {
    if (packable(a)) return choose<T, KT, 256, 2>(cap);
  }
  return choose<T, KT, 128, 1>(cap);
}

}  // namespace

GqaChoice pick_decode_gqa(const fa_attn_args& a) {
  const GqaChoice none{nullptr, 0, 1};
  if (a.heads_k <= 0 || a.heads_q % a.heads_k) return none;
  // One query row per request: groups of DECODE_GQA_MIN_GROUP or more (the
  // VALU kernel is faster below); 2..DECODE_GQA_MAX_ROWS rows: any group
  // (nothing else runs a few rows per request as decode).
  if (a.max_seqlen_q > DECODE_GQA_MAX_ROWS) return none;
  if (a.max_seqlen_q <= 1 && a.heads_q / a.heads_k < DECODE_GQA_MIN_GROUP && !(a.head_dim_qk == 64 && packable(a)))
    return none;
  if (a.q_dtype != FA_BF16 && a.q_dtype != FA_F16) return none;
  // P.V runs on probabilities rounded to the query's type: fp32 outputs
  // (held to fp32 accuracy) take the VALU kernel, which keeps P in fp32.
  if (a.out_dtype != a.q_dtype) return none;
  if (a.k_dtype != a.v_dtype || (a.k_dtype != a.q_dtype && a.k_dtype != FA_E4M3)) return none;
  if (a.head_dim_qk != a.head_dim_v || (a.head_dim_qk != 64 && a.head_dim_qk != 128)) return none;
  if (a.alibi || a.mask_kind != 0) return none;
  if (a.page_size && a.page_size % 16) return none;
  const int kvb = a.k_dtype == FA_E4M3 ? 1 : 2;
  if (!chunks_aligned(a, kvb)) return none;
  // Row and page offsets are 32-bit byte counts in the kernel's addressing.
  for (int i = 0; i < 2; ++i)
    if (a.k_stride[i] * kvb >= (1ll << 31) / 16 || a.v_stride[i] * kvb >= (1ll << 31) / 16) return none;
  const bool cap = a.softcap > 0.0f, fp8 = a.k_dtype == FA_E4M3;
  if (a.q_dtype == FA_BF16) return fp8 ? choose_dim<BF16T, E4M3T>(a, cap) : choose_dim<BF16T, BF16T>(a, cap);
  return fp8 ? choose_dim<F16T, E4M3T>(a, cap) : choose_dim<F16T, F16T>(a, cap);
}

}  // namespace fa_decode
