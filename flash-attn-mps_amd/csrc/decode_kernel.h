// Single-query split-KV decode over packed or paged K/V, plus the split merge.
//
// Semantics follow flash_attn_mps/_decode.py:40-99 and
// flash_attn_mps/kernels/attention_decode.metal:18-207: one query per request,
// keys [vis_begin, len) with vis_begin = len - window_left - 1 under a left
// window, scores scaled by softmax_scale * q_descale * k_descale, softcap on
// the scaled score, the sink seeding (max, sum) = (sink, 1) of split 0 only,
// the output multiplied by v_descale, fp32 partial states merged by
// log-sum-exp.
//
// gfx950 layout.  A workgroup (4 waves) owns one (request, group of GT query
// heads sharing a KV head, split of `span` keys).  Every 16-lane row of a wave
// owns NT consecutive key positions per step and spreads the head dimension
// over its 16 lanes, so a 256-byte K or V head row is one coalesced 16-lane
// access of 16-byte loads.  A wave step covers 4 rows x NT positions; the
// wave's next step is STEP * 4 positions further (the 4 waves interleave).
// * The K/V loads of step t+1 are issued before step t is computed (two
//   register buffers), so every wave keeps one step of K/V in flight while
//   it does arithmetic.
// * Block-table entries for 64 steps are loaded once per wave into lanes
//   (lane 4u + row holds the page of step u's row) and handed to the rows
//   with ds_bpermute: no dependent table load inside the loop.
// * Loads are unconditional: positions outside the split clamp to the row's
//   first/last valid position (rows with none read the split's first key),
//   and their scores are masked to -inf, so V is finite and p = 0.
// * Q.K runs on packed pairs with v_dot2_f32_bf16 / v_dot2_f32_f16 (FP8 K
//   converts exactly to the query's 16-bit type with v_cvt_scalef32_pk_*);
//   the softmax scale is applied to the reduced score.  P.V is fp32 FMA.
// * exp2 online softmax per row whose running max moves only when a step
//   raises it by more than 2^8 (probabilities stay <= 256); rows combine
//   with lane shuffles and waves through LDS at the end.
#pragma once
#include "attn_common.h"

namespace fa_decode {

constexpr int DEC_THREADS = 256;
constexpr int DEC_PAGE_ALIGN = 8;   // paged K/V needs P % 8 == 0
#ifndef FA_DEC_MINB
#define FA_DEC_MINB 2
#endif
constexpr float DEC_RESCALE = 8.0f;

typedef __attribute__((ext_vector_type(2))) __bf16 dec_bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 dec_f16x2;

// Positions per 16-lane row per step: 4, or 2 for K+V row pairs of 64 bytes
// per lane or more (keeps two register buffers within budget).
template <int KB, int VB>
struct DecodeRows {
  static constexpr int value = KB + VB >= 64 ? 2 : 4;
};

template <int BYTES>
struct LoadChunk {
  static constexpr int value = BYTES % 16 == 0 ? 16 : BYTES % 8 == 0 ? 8 : 4;
};

// Lane layout of a K or V row: a lane's BYTES are split into pieces of 16,
// 8 or 4 bytes (largest first), and piece j of lane l sits at byte
// 16 * start(j) + size(j) * l of the row, so each piece is one load
// instruction over a contiguous span of the 16-lane row (a bf16 192-dim
// row: 16 bytes at 16 l, then 8 bytes at 256 + 8 l, instead of three
// 8-byte loads at a 24-byte lane stride; a bf16 256-dim row: 16 bytes at
// 16 l and at 256 + 16 l).  The query takes the K row's element layout;
// the output dims follow the V row's.
constexpr int piece_bytes(int total, int j) {
  int rem = total;
  for (int i = 0; rem > 0; ++i) {
    const int s = rem >= 16 ? 16 : rem >= 8 ? 8 : 4;
    if (i == j) return s;
    rem -= s;
  }
  return 0;
}
constexpr int piece_count(int total) {
  int n = 0;
  while (piece_bytes(total, n) > 0) ++n;
  return n;
}
constexpr int piece_start(int total, int j) {
  int s = 0;
  for (int i = 0; i < j; ++i) s += piece_bytes(total, i);
  return s;
}

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

// Non-temporal vector types for the K/V stream (each cache row is read once
// per call).
typedef __attribute__((ext_vector_type(4))) uint32_t dec_u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t dec_u32x2;

// A lane's pieces of a K or V row (non-temporal): off[j] = the lane's byte
// offset of piece j inside the row.
template <int BYTES>
FA_DEV void load_pieces_nt(const char* row, const uint32_t (&off)[piece_count(BYTES)], uint32_t (&w)[BYTES / 4]) {
#pragma unroll
  for (int j = 0; j < piece_count(BYTES); ++j) {
    const char* p = row + off[j];
    const int w0 = piece_start(BYTES, j) / 4;
    if (piece_bytes(BYTES, j) == 16) {
      const dec_u32x4 v = __builtin_nontemporal_load((const dec_u32x4*)p);
      w[w0] = v[0]; w[w0 + 1] = v[1]; w[w0 + 2] = v[2]; w[w0 + 3] = v[3];
    } else if (piece_bytes(BYTES, j) == 8) {
      const dec_u32x2 v = __builtin_nontemporal_load((const dec_u32x2*)p);
      w[w0] = v[0]; w[w0 + 1] = v[1];
    } else {
      w[w0] = __builtin_nontemporal_load((const uint32_t*)p);
    }
  }
}

// s_waitcnt vmcnt(N): every vector-memory load but the N most recent has
// returned (loads return in order).
template <int N>
FA_DEV void wait_older_than() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
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
  } else {
    static_assert(T::id == FA_E4M3, "V element type");
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
      f[4 * i] = lo[0]; f[4 * i + 1] = lo[1]; f[4 * i + 2] = hi[0]; f[4 * i + 3] = hi[1];
    }
  }
}

// c + a.lo * b.lo + a.hi * b.hi on packed 16-bit pairs, fp32 result.
template <typename CT> FA_DEV float dot2(uint32_t a, uint32_t b, float c);
template <> FA_DEV float dot2<BF16T>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dec_bf16x2, a), __builtin_bit_cast(dec_bf16x2, b), c, false);
}
template <> FA_DEV float dot2<F16T>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(dec_f16x2, a), __builtin_bit_cast(dec_f16x2, b), c, false);
}

// K row words -> EK/2 packed pairs of the compute type (FP8 widens exactly).
template <typename CT, typename KT, int EK>
FA_DEV void k_pairs(const uint32_t* w, uint32_t* p) {
  if constexpr (KT::id == FA_E4M3) {
#pragma unroll
    for (int i = 0; i < EK / 4; ++i) {
      if constexpr (CT::id == FA_BF16) {
        p[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[i], 1.0f, false));
        p[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[i], 1.0f, true));
      } else {
        p[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[i], 1.0f, false));
        p[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[i], 1.0f, true));
      }
    }
  } else {
    static_assert(KT::id == CT::id, "16-bit K must match the compute type");
#pragma unroll
    for (int i = 0; i < EK / 2; ++i) p[i] = w[i];
  }
}

template <typename CT>
FA_DEV uint32_t pack_pair_bits(float lo, float hi) {
  if constexpr (CT::id == FA_BF16) return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
  else return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
}

// First key any of a request's q_len query rows sees (the rows are the last
// q_len positions; a left window starts at the first row's position - WL).
FA_DEV int decode_vis_begin(const fa_attn_args& a, int k_len, int q_len = 1) {
  return a.window_left >= 0 ? max(0, k_len - q_len - a.window_left) : 0;
}

// Work order of the split workgroups (both decode kernels).  The grid
// holds num_splits x batch slots per head tile; slot w = blockIdx.y +
// num_splits blockIdx.z takes, longest first: every split of a full span of
// keys, request by request, then each request's last, shorter split by
// decreasing length class (span / 16 keys per class; a request with no
// visible key has one empty split, class 0), and past the work the slots
// exit at once.  In plain (split, request) order a request's unused split
// slots sit among the work (each one a workgroup launch), and the short last
// splits fall anywhere, so the launch can end on a few full splits started
// late: measured on config 3 (64 requests, 512-32768 keys) the plain order
// ran ~4% longer.  Requests outside 1..rows query rows get no slot, as the
// merge expects, and no request gets a split past num_splits - 1.  Every
// wave computes the same item from the request metadata (up to
// SPLIT_ORDER_CHUNKS x 64 requests, one per lane and chunk, in registers);
// the chosen request's RequestInfo comes from the lane that loaded it.
// Larger batches keep the grid order (split y, request z).
constexpr int SPLIT_ORDER_CHUNKS = 4;
constexpr int SPLIT_CLASSES = 16;

struct SplitItem {
  RequestInfo r;
  int64_t b;
  int split;
  bool ok;
};

FA_DEV RequestInfo request_from_lane(const RequestInfo& r, int l) {
  RequestInfo o;
  o.q_begin = __builtin_amdgcn_readlane(r.q_begin, l);
  o.q_len = __builtin_amdgcn_readlane(r.q_len, l);
  o.k_len = __builtin_amdgcn_readlane(r.k_len, l);
  o.k_base = __builtin_amdgcn_readlane(r.k_base, l);
  o.left = __builtin_amdgcn_readlane(r.left, l);
  o.causal = __builtin_amdgcn_readlane((int)r.causal, l) != 0;
  return o;
}

FA_DEV SplitItem split_item(const fa_attn_args& a, int rows, int span) {
  const int S = a.num_splits;
  SplitItem it;
  it.ok = false;
  it.b = 0;
  it.split = 0;
  if (a.batch > 64 * SPLIT_ORDER_CHUNKS) {
    it.split = blockIdx.y;
    it.b = blockIdx.z;
    it.r = load_request(a, it.b);
    it.ok = it.r.q_len >= 1 && it.r.q_len <= rows;
    return it;
  }
  const int w = (int)(blockIdx.y + gridDim.y * blockIdx.z);
  const int lane = threadIdx.x & 63;
  const int B = (int)a.batch, nc = (B + 63) / 64;
  RequestInfo rq[SPLIT_ORDER_CHUNKS];
  int full[SPLIT_ORDER_CHUNKS], cls[SPLIT_ORDER_CHUNKS];
#pragma unroll
  for (int c = 0; c < SPLIT_ORDER_CHUNKS; ++c) {
    full[c] = 0;
    cls[c] = -1;
    rq[c] = RequestInfo{0, 0, 0, 0, 0, false};
    const int q = 64 * c + lane;
    if (c < nc && q < B) {
      rq[c] = load_request(a, q);
      if (rq[c].q_len >= 1 && rq[c].q_len <= rows) {
        const int n = max(rq[c].k_len - decode_vis_begin(a, rq[c].k_len, rq[c].q_len), 0);
        full[c] = min(n / span, S);
        const int rem = n - full[c] * span;
        if ((rem > 0 || n == 0) && full[c] < S) cls[c] = (int)((int64_t)rem * SPLIT_CLASSES / span);
      }
    }
  }
  // Full splits: the request whose running count passes w.
  int base = 0;
#pragma unroll
  for (int c = 0; c < SPLIT_ORDER_CHUNKS; ++c) {
    int incl = full[c];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(incl, o);
      if (lane >= o) incl += t;
    }
    const uint64_t hit = __ballot(w < base + incl);
    if (hit) {
      const int l = __builtin_ctzll(hit);
      it.r = request_from_lane(rq[c], l);
      it.b = 64 * c + l;
      it.split = w - base - (__builtin_amdgcn_readlane(incl, l) - __builtin_amdgcn_readlane(full[c], l));
      it.ok = true;
      return it;
    }
    base += __builtin_amdgcn_readlane(incl, 63);
  }
  // Last splits: longest class first, requests in order within a class.
  int rest = w - base;
  int k = SPLIT_CLASSES - 1;
  for (; k >= 0; --k) {
    int n = 0;
#pragma unroll
    for (int c = 0; c < SPLIT_ORDER_CHUNKS; ++c) n += __popcll(__ballot(cls[c] == k));
    if (rest < n) break;
    rest -= n;
  }
  if (k < 0) return it;
#pragma unroll
  for (int c = 0; c < SPLIT_ORDER_CHUNKS; ++c) {
    const uint64_t m = __ballot(cls[c] == k);
    const int n = __popcll(m);
    if (rest < n) {
      const uint64_t below = lane ? m & (~0ull >> (64 - lane)) : 0ull;
      const int l = __builtin_ctzll(__ballot(cls[c] == k && __popcll(below) == rest));
      it.r = request_from_lane(rq[c], l);
      it.b = 64 * c + l;
      it.split = __builtin_amdgcn_readlane(full[c], l);
      it.ok = true;
      return it;
    }
    rest -= n;
  }
  return it;
}

// D / DV: the tile's head dims; DT / DVT <= them: the tensors' own.  Lanes
// past the real dims read the row's last real chunk (always in bounds), with
// a zero query there, so they add nothing to Q.K; their V columns are never
// stored.
// PK = 2: two neighbouring KV heads, whose rows sit next to each other in
// every key row, run in one workgroup: every lane loads its pieces of both
// heads' rows (the second head's one head row further on), so a 16-lane
// row's loads of one key cover both rows back to back, twice the run of one
// head.  A lane's words hold the first head's pieces, then the second's,
// each in its own head's layout: query head g of the workgroup (heads of
// the first KV head, then of the second) takes the K and V words of its half
// only, and the arithmetic per byte is that of one head.  GT counts the
// query heads of both halves.
template <typename CT, typename KT, typename VT, int D, int DV, int GT, bool CAP, int DT = D, int DVT = DV,
          bool ALIBI = false, int PK = 1>
__global__ __launch_bounds__(DEC_THREADS, FA_DEC_MINB) void decode_kernel(const fa_attn_args a, const int span) {
  constexpr int EK = D / 16, EV = DV / 16;
  constexpr int LK = DT / EK, LV = DVT / EV;   // lanes of a 16-lane row holding real dims
  static_assert(DT % EK == 0 && DVT % EV == 0 && DT <= D && DVT <= DV, "true head dims fill whole lane chunks");
  constexpr int KB = EK * KT::bytes, VB = EV * VT::bytes;   // one head's bytes per lane
  static_assert(PK == 1 || (PK == 2 && DT == D && DVT == DV && GT % 2 == 0), "paired heads: unpadded rows");
  constexpr int KBP = PK * KB, VBP = PK * VB;   // bytes per lane of the (paired) row
  constexpr int GH = GT / PK;                   // query heads per KV head of the workgroup
  constexpr int NT = DecodeRows<KBP, VBP>::value;
  constexpr int STEP = 4 * NT;          // positions of one wave step
  constexpr int WSTRIDE = 4 * STEP;     // positions between a wave's consecutive steps
  static_assert(EK % 4 == 0 && EV % 4 == 0 && KB % 4 == 0 && VB % 4 == 0, "decode tile shape");
  static_assert(LK == 16 || piece_count(KB) == 1, "padded K rows use a single piece per lane");
  static_assert(LV == 16 || piece_count(VB) == 1, "padded V rows use a single piece per lane");
  __shared__ float sm_m[4][GT], sm_l[4][GT];
  __shared__ float sm_acc[4][GT][DV];
  // Half of the paired row that query head g of the workgroup reads.
  auto half_of = [](int g) { return PK > 1 ? g / GH : 0; };

  // Head groups are the fastest grid dimension: the workgroups of one
  // (request, split) run together and read whole token rows of the same pages;
  // split_item() gives each (split, request) slot its work.
  // The wave index as a scalar: everything the steps derive from it (their
  // positions, whether a step lies wholly inside the split) is then
  // wave-uniform, so the full / partial load paths are scalar branches
  // rather than exec-masked ones the compiler would run back to back (and
  // whose merged loads made it wait for most of the next step's loads
  // before computing the current one).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, rg = lane >> 4, l16 = lane & 15;
  const SplitItem item = split_item(a, 1, span);
  if (!item.ok) return;
  const int split = item.split;
  const int64_t b = item.b;
  const RequestInfo r = item.r;
  // Workgroup x holds query heads t GT .. t GT + GT - 1 of KV head kh's group
  // (t = x % tiles, tiles = ceil(group / GT)); a last tile past the group
  // recomputes its last real head in the spare slots and stores nothing there.
  // Paired (PK = 2): kh numbers KV head pairs, whose PK groups are one
  // group of contiguous query heads, held whole by the workgroup (GT = PK x
  // the heads per KV head).
  const int group = PK * (int)(a.heads_q / a.heads_k), tiles = (group + GT - 1) / GT;
  const int kh = blockIdx.x / tiles, t0 = (blockIdx.x % tiles) * GT;
  const int h0 = kh * group + t0, nreal = min(GT, group - t0);
  const int vis_begin = decode_vis_begin(a, r.k_len);
  const int begin = vis_begin + split * span;
  const int end = min(r.k_len, begin + span);
  if (split > 0 && begin >= end) return;
  const int64_t tq = r.q_begin;
  const int S = a.num_splits;

  // Descales per KV head (of each half when paired).
  float sscale[PK], vscale[PK];
#pragma unroll
  for (int u = 0; u < PK; ++u) {
    const int kv = PK * kh + u;
    sscale[u] = a.softmax_scale * descale_of(a.q_descale, a.q_descale_stride, b, kv) *
                descale_of(a.k_descale, a.k_descale_stride, b, kv) * (CAP ? 1.0f : LOG2E);
    vscale[u] = descale_of(a.v_descale, a.v_descale_stride, b, kv);
  }
  const float cap_in = CAP ? 2.0f * LOG2E / a.softcap : 0.0f, cap_out = a.softcap * LOG2E;
  // ALiBi: -slope |q_pos - key| in log2 units after the softcap
  // (flash_attn_mps/kernels/attention.metal:47-51); the query sits at key
  // position k_len - 1, storage row qrow, so the bias is slope (row - qrow).
  // The slopes are wave-uniform: kept in scalar registers.  A template flag,
  // so kernels without ALiBi keep their registers (a runtime test cost the
  // eight-head tiles 7%).
  float slope2[GT];
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    const float sl =
        ALIBI ? a.alibi[b * a.alibi_stride[0] + (int64_t)(h0 + min(g, nreal - 1)) * a.alibi_stride[1]] * LOG2E : 0.0f;
    slope2[g] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sl)));
  }
  const int qrow = r.k_base + r.left + r.k_len - 1;

  // Query pairs of this lane's dims (the K row's piece layout), unscaled, in
  // the compute type.  Piece j holds EP_j = size(j) / KT::bytes elements,
  // dims 16 E_j + EP_j lq .. + EP_j (E_j = elements before piece j).
  const int lq = min(l16, LK - 1);
  uint32_t qp[GT][EK / 2];
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    const int64_t q0 = tq * a.q_stride[0] + (int64_t)(h0 + min(g, nreal - 1)) * a.q_stride[1];
#pragma unroll
    for (int j = 0; j < piece_count(KB); ++j) {
      const int ep = piece_bytes(KB, j) / KT::bytes, e0 = piece_start(KB, j) / KT::bytes;
      const int d0 = 16 * e0 + ep * lq;
      uint32_t* dst = qp[g] + e0 / 2;
      if (a.q_stride[2] == 1) {
        const char* src = (const char*)a.q + (q0 + d0) * 2;
        if (ep == 8) {
          uint32_t w[4];
          load_words<16>(src, w);
          for (int i = 0; i < 4; ++i) dst[i] = w[i];
        } else if (ep == 4) {
          uint32_t w[2];
          load_words<8>(src, w);
          for (int i = 0; i < 2; ++i) dst[i] = w[i];
        } else {
          uint32_t w[8];
          load_words<32>(src, w);
          for (int i = 0; i < 8; ++i) dst[i] = w[i];
        }
      } else {
        for (int i = 0; i < ep / 2; ++i)
          dst[i] = pack_pair_bits<CT>(load_elem<CT>(a.q, q0 + (int64_t)(d0 + 2 * i) * a.q_stride[2]),
                                      load_elem<CT>(a.q, q0 + (int64_t)(d0 + 2 * i + 1) * a.q_stride[2]));
      }
    }
    if (LK < 16 && l16 >= LK) {
#pragma unroll
      for (int j = 0; j < EK / 2; ++j) qp[g][j] = 0u;   // padding dims: no contribution to Q.K
    }
  }

  float m[GT], l[GT], acc[GT][EV];
  const bool seed = a.sinks && split == 0 && wave == 0 && rg == 0;
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    m[g] = seed ? a.sinks[(int64_t)(h0 + min(g, nreal - 1)) * a.sink_stride] * LOG2E : -INFINITY;
    l[g] = seed ? 1.0f : 0.0f;
#pragma unroll
    for (int e = 0; e < EV; ++e) acc[g][e] = 0.0f;
  }

  // Storage positions [plo, phi) of this split (packed rows or paged slots).
  const int plo = r.k_base + r.left + begin, phi = r.k_base + r.left + end;
  const int P = (int)a.page_size;
  const int sb0 = (plo & ~(STEP - 1)) + STEP * wave;
  const int nsteps = (begin < end && sb0 < phi) ? (phi - 1 - sb0) / WSTRIDE + 1 : 0;

  // Byte addressing.  Row r of page blk of KV head kh, dims from l16 * E:
  // base + blk * page_stride + r * row_stride + kh * head_stride + l16 * E * bytes.
  const uint32_t kpage_b = (uint32_t)(a.k_stride[0] * KT::bytes), vpage_b = (uint32_t)(a.v_stride[0] * VT::bytes);
  const uint32_t krow_b = (uint32_t)(a.k_stride[1] * KT::bytes), vrow_b = (uint32_t)(a.v_stride[1] * VT::bytes);
  const char* kbase = (const char*)a.k + (int64_t)(PK * kh) * a.k_stride[2] * KT::bytes;
  uint32_t koff[piece_count(KB)];
#pragma unroll
  for (int j = 0; j < piece_count(KB); ++j) koff[j] = 16 * piece_start(KB, j) + piece_bytes(KB, j) * lq;
  const char* vbase = (const char*)a.v + (int64_t)(PK * kh) * a.v_stride[2] * VT::bytes;
  const int lv = min(l16, LV - 1);
  uint32_t voff[piece_count(VB)];
#pragma unroll
  for (int j = 0; j < piece_count(VB); ++j) voff[j] = 16 * piece_start(VB, j) + piece_bytes(VB, j) * lv;
  // Paired: the second head's row, one head stride further.
  const uint32_t khead_b = (uint32_t)(a.k_stride[2] * KT::bytes), vhead_b = (uint32_t)(a.v_stride[2] * VT::bytes);

  // Address of the split's first key: the read target of rows with no valid position.
  const char* ksafe = kbase;
  const char* vsafe = vbase;
  if (nsteps > 0) {
    if (P) {
      const uint32_t blk = (uint32_t)load_invariant_i32(a.block_table, b * a.bt_stride[0] + (int64_t)(plo / P) * a.bt_stride[1]);
      ksafe += (uint64_t)blk * kpage_b + (uint64_t)(plo % P) * krow_b;
      vsafe += (uint64_t)blk * vpage_b + (uint64_t)(plo % P) * vrow_b;
    } else {
      ksafe += (uint64_t)plo * krow_b;
      vsafe += (uint64_t)plo * vrow_b;
    }
  }

  // Pages: a wave step covers STEP consecutive positions from sbt (a
  // multiple of STEP) and P is a multiple of 8, so the step's positions
  // inside the split lie in at most two pages, A and B, and each row's NT
  // positions in one of them.  Their block-table entries are read through
  // the scalar cache (wave-uniform addresses, tracked apart from the K/V
  // loads, so waiting for them never waits for K/V).  Pages are taken of
  // positions clamped into the split, so the table is read in bounds.
  const int lp = (P > 0 && (P & (P - 1)) == 0) ? 31 - __builtin_clz(P) : -1;
  auto page_of = [&](int pos) { return lp >= 0 ? pos >> lp : pos / P; };

  // Row state advanced once per issued step: paged -> row index inside the
  // page (and its byte offsets); packed -> byte offsets of the row itself.
  const int rp0 = sb0 + NT * rg;
  int inr = P ? rp0 % P : 0;
  const int wrap = P ? WSTRIDE % P : 0;
  uint64_t kin = P ? (uint64_t)inr * krow_b : (uint64_t)rp0 * krow_b;
  uint64_t vin = P ? (uint64_t)inr * vrow_b : (uint64_t)rp0 * vrow_b;
  const uint64_t kstep_packed = (uint64_t)WSTRIDE * krow_b, vstep_packed = (uint64_t)WSTRIDE * vrow_b;

  // One load site per buffer: a step wholly inside the split reads positions
  // rp .. rp + NT - 1 of each row; otherwise each row clamps them into the
  // split (rows with none read the split's first key).  The choice is a
  // scalar branch that only sets offsets, so the loads of consecutive steps
  // never alias registers the compiler must wait on.
  auto issue = [&](int t, uint32_t (&kw)[NT][KBP / 4], uint32_t (&vw)[NT][VBP / 4]) {
    const int sbt = sb0 + WSTRIDE * t;
    const bool full = sbt >= plo && sbt + STEP <= phi;
    const char* krow = kbase + kin;
    const char* vrow = vbase + vin;
    const int rp = rp0 + WSTRIDE * t;
    if (P) {
      const int pa = page_of(min(max(sbt, plo), phi - 1)), pb = page_of(min(max(sbt + STEP - 1, plo), phi - 1));
      const int64_t trow = b * a.bt_stride[0];
      const uint32_t ba = (uint32_t)load_invariant_i32(a.block_table, trow + (int64_t)pa * a.bt_stride[1]);
      const uint32_t bb = (uint32_t)load_invariant_i32(a.block_table, trow + (int64_t)pb * a.bt_stride[1]);
      const uint32_t blk = rp >= pb * P ? bb : ba;
      krow += (uint64_t)blk * kpage_b;
      vrow += (uint64_t)blk * vpage_b;
    }
    uint32_t ko[NT], vo[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      ko[i] = (uint32_t)i * krow_b;
      vo[i] = (uint32_t)i * vrow_b;
    }
    if (!full) {
      const bool row_ok = rp + NT > plo && rp < phi;
      const int lo_i = row_ok ? max(plo - rp, 0) : 0;
      const int hi_i = row_ok ? min(phi - rp, NT) - 1 : 0;
      if (!row_ok) {
        krow = ksafe;
        vrow = vsafe;
      }
#pragma unroll
      for (int i = 0; i < NT; ++i) {
        const uint32_t j = (uint32_t)min(max(i, lo_i), hi_i);
        ko[i] = j * krow_b;
        vo[i] = j * vrow_b;
      }
    }
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
      for (int u = 0; u < PK; ++u)
        load_pieces_nt<KB>(krow + ko[i] + u * khead_b, koff, *(uint32_t(*)[KB / 4])(kw[i] + u * (KB / 4)));
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
      for (int u = 0; u < PK; ++u)
        load_pieces_nt<VB>(vrow + vo[i] + u * vhead_b, voff, *(uint32_t(*)[VB / 4])(vw[i] + u * (VB / 4)));
    if (P) {
      inr += wrap;
      kin += (uint64_t)wrap * krow_b;
      vin += (uint64_t)wrap * vrow_b;
      if (inr >= P) {
        inr -= P;
        kin -= (uint64_t)P * krow_b;
        vin -= (uint64_t)P * vrow_b;
      }
    } else {
      kin += kstep_packed;
      vin += vstep_packed;
    }
  };

  auto compute = [&](int t, const uint32_t (&kw)[NT][KBP / 4], const uint32_t (&vw)[NT][VBP / 4]) {
    const int sbt = sb0 + WSTRIDE * t;
    const bool full = sbt >= plo && sbt + STEP <= phi;
    const int rp = rp0 + WSTRIDE * t;
    float s[GT][NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      uint32_t kp[PK * EK / 2];
      k_pairs<CT, KT, PK * EK>(kw[i], kp);
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        float dot = 0.0f;
#pragma unroll
        for (int j = 0; j < EK / 2; ++j) dot = dot2<CT>(qp[g][j], kp[half_of(g) * (EK / 2) + j], dot);
        s[g][i] = dot;
      }
    }
#pragma unroll
    for (int g = 0; g < GT; ++g)
#pragma unroll
      for (int i = 0; i < NT; ++i) {
        float v = row16_sum(s[g][i]) * sscale[half_of(g)];
        if constexpr (CAP) v = cap_out * (1.0f - 2.0f * __builtin_amdgcn_rcpf(fast_exp2(v * cap_in) + 1.0f));
        if constexpr (ALIBI) v = fmaf(slope2[g], (float)(rp + i - qrow), v);
        s[g][i] = v;
      }
    if (!full) {
#pragma unroll
      for (int i = 0; i < NT; ++i) {
        const bool ok = rp + i >= plo && rp + i < phi;
#pragma unroll
        for (int g = 0; g < GT; ++g) s[g][i] = ok ? s[g][i] : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      float mx = s[g][0];
#pragma unroll
      for (int i = 1; i < NT; ++i) mx = fmaxf(mx, s[g][i]);
      const bool need = mx > m[g] + DEC_RESCALE;
      if (__builtin_expect(__any(need), 0)) {
        const float f = need ? fast_exp2(m[g] - mx) : 1.0f;
        if (need) m[g] = mx;
        l[g] *= f;
#pragma unroll
        for (int e = 0; e < EV; ++e) acc[g][e] *= f;
      }
      const float ref = m[g] == -INFINITY ? 0.0f : m[g];
      float sum = 0.0f;
#pragma unroll
      for (int i = 0; i < NT; ++i) {
        s[g][i] = fast_exp2(s[g][i] - ref);
        sum += s[g][i];
      }
      l[g] += sum;
    }
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      float vf[PK * EV];
      words_to_f32<VT, PK * EV>(vw[i], vf);
#pragma unroll
      for (int g = 0; g < GT; ++g)
#pragma unroll
        for (int e = 0; e < EV; ++e) acc[g][e] = fmaf(s[g][i], vf[half_of(g) * EV + e], acc[g][e]);
    }
  };

  if (nsteps > 0) {
    uint32_t kwa[NT][KBP / 4], vwa[NT][VBP / 4], kwb[NT][KBP / 4], vwb[NT][VBP / 4];
    // Steps t + 1 and t + 2 are issued unconditionally (past the last step
    // they read the split's first key: one K and one V row per wave,
    // cached) and only the compute of step t + 1 is conditional, so the loop
    // has one exit, at the bottom.  With exits after each compute (and a
    // conditional issue before), the compiler's wait analysis put an
    // s_waitcnt vmcnt(0) at the loop head, draining the step in flight once
    // every two steps; in this form the next step's loads stay in flight
    // throughout.
    issue(0, kwa, vwa);
    for (int t = 0; t < nsteps; t += 2) {
      issue(t + 1, kwb, vwb);
      compute(t, kwa, vwa);
      issue(t + 2, kwa, vwa);
      if (t + 1 < nsteps) compute(t + 1, kwb, vwb);
    }
    wait_older_than<0>();
  }

  // Combine the four 16-lane rows of the wave (same l16 <-> same dims; the V
  // row's piece layout: element e of piece j is dim 16 E_j + EP_j l16 + e - E_j).
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
      for (int j = 0; j < piece_count(VB); ++j) {
        const int ep = piece_bytes(VB, j) / VT::bytes, e0 = piece_start(VB, j) / VT::bytes;
#pragma unroll
        for (int e = 0; e < ep; ++e) sm_acc[wave][g][16 * e0 + ep * l16 + e] = acc[g][e0 + e];
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < nreal * DVT; idx += DEC_THREADS) {
    const int g = idx / DVT, d = idx - g * DVT;
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
    const float norm = L > 0.0f ? vscale[half_of(g)] / L : 0.0f;
    const float lse = L > 0.0f ? M * LN2 + logf(L) : -INFINITY;
    const int h = h0 + g;
    if (S == 1) {
      store_any(a.out, tq * a.out_stride[0] + (int64_t)h * a.out_stride[1] + (int64_t)d * a.out_stride[2], a.out_dtype,
                O * norm);
      if (d == 0) a.lse[(int64_t)h * a.lse_stride[0] + tq * a.lse_stride[1]] = lse;
    } else {
      // Partial outputs [batch][S][Hq][Dv], LSEs [batch][Hq][S], as the
      // matrix-core decode writes them (streaming stores, split-major rows).
      __builtin_nontemporal_store(O * norm, &a.partial_out[((b * S + split) * a.heads_q + h) * DVT + d]);
      if (d == 0) a.partial_lse[(b * a.heads_q + h) * S + split] = lse;
    }
  }
}

using DecodeKernel = void (*)(fa_attn_args, int);

template <typename CT, typename KT, typename VT, int D, int DV, bool CAP, bool ALIBI, int DT = D, int DVT = DV>
DecodeKernel pick_group(int gt) {
  switch (gt) {
    case 8: if constexpr (D == 128 && DV == 128) return decode_kernel<CT, KT, VT, D, DV, 8, CAP, DT, DVT, ALIBI>; else return nullptr;
    case 4: if constexpr (4 * (D + DV) <= 64 * 16) return decode_kernel<CT, KT, VT, D, DV, 4, CAP, DT, DVT, ALIBI>; else return nullptr;
    case 2: if constexpr (2 * (D + DV) <= 64 * 16) return decode_kernel<CT, KT, VT, D, DV, 2, CAP, DT, DVT, ALIBI>; else return nullptr;
    case 1: return decode_kernel<CT, KT, VT, D, DV, 1, CAP, DT, DVT, ALIBI>;
    default: return nullptr;
  }
}

// Head dims 32 and 72/80/96 (dq == dv) run in the 64- and 128-dim tiles.
template <typename CT, typename KT, typename VT, bool CAP, bool ALIBI>
DecodeKernel pick_dims_cap(int64_t d, int64_t dv, int gt) {
  if (d == 192 && dv == 128) return pick_group<CT, KT, VT, 192, 128, CAP, ALIBI>(gt);
  if (d != dv) return nullptr;
  switch (d) {
    case 32: return pick_group<CT, KT, VT, 64, 64, CAP, ALIBI, 32, 32>(gt);
    case 64: return pick_group<CT, KT, VT, 64, 64, CAP, ALIBI>(gt);
    case 72: return pick_group<CT, KT, VT, 128, 128, CAP, ALIBI, 72, 72>(gt);
    case 80: return pick_group<CT, KT, VT, 128, 128, CAP, ALIBI, 80, 80>(gt);
    case 96: return pick_group<CT, KT, VT, 128, 128, CAP, ALIBI, 96, 96>(gt);
    case 128: return pick_group<CT, KT, VT, 128, 128, CAP, ALIBI>(gt);
    case 256: return pick_group<CT, KT, VT, 256, 256, CAP, ALIBI>(gt);
    default: return nullptr;
  }
}

// The tile head dim a tensor head dim runs in (0: none).
inline int64_t decode_tile_dim(int64_t d) {
  switch (d) {
    case 32: case 64: return 64;
    case 72: case 80: case 96: case 128: return 128;
    case 192: return 192;
    case 256: return 256;
    default: return 0;
  }
}

// Paired KV heads (PK = 2), 2 x the group's heads per workgroup: E4M3 d128
// (groups of 1-2) and 16-bit 192/128 (groups of 1), the layouts where
// pairing measured faster (valu_pair in decode_kernel.hip).
template <typename CT, typename KT, typename VT, bool CAP>
DecodeKernel pick_pair(int64_t d, int64_t dv, int gt) {
  if constexpr (KT::bytes == 1) {
    if (d == 128 && dv == 128) {
      if (gt == 2) return decode_kernel<CT, KT, VT, 128, 128, 2, CAP, 128, 128, false, 2>;
      if (gt == 4) return decode_kernel<CT, KT, VT, 128, 128, 4, CAP, 128, 128, false, 2>;
    }
  } else {
    if (d == 192 && dv == 128 && gt == 2) return decode_kernel<CT, KT, VT, 192, 128, 2, CAP, 192, 128, false, 2>;
  }
  return nullptr;
}

template <typename CT, typename KT, typename VT>
DecodeKernel pick_dims(int64_t d, int64_t dv, int gt, bool cap, bool alibi, int pk) {
  if (pk == 2) {
    if (alibi) return nullptr;
    return cap ? pick_pair<CT, KT, VT, true>(d, dv, gt) : pick_pair<CT, KT, VT, false>(d, dv, gt);
  }
  // ALiBi variants exist without softcap only (softcap + ALiBi: generic kernel).
  if (alibi) return cap ? nullptr : pick_dims_cap<CT, KT, VT, false, true>(d, dv, gt);
  return cap ? pick_dims_cap<CT, KT, VT, true, false>(d, dv, gt) : pick_dims_cap<CT, KT, VT, false, false>(d, dv, gt);
}

// Variants by (query, K/V) types, instantiated in decode_inst_*.hip so they
// compile in parallel.
DecodeKernel pick_decode_bf16(int64_t d, int64_t dv, int gt, bool cap, bool alibi, int pk);
DecodeKernel pick_decode_f16(int64_t d, int64_t dv, int gt, bool cap, bool alibi, int pk);
DecodeKernel pick_decode_fp8_bf16(int64_t d, int64_t dv, int gt, bool cap, bool alibi, int pk);
DecodeKernel pick_decode_fp8_f16(int64_t d, int64_t dv, int gt, bool cap, bool alibi, int pk);

// The matrix-core decode for GQA groups of DECODE_GQA_MIN_GROUP or more query
// heads per KV head, and for any group when 64-dim KV heads run in pairs
// (decode_gqa.h, decode_gqa.hip): its kernel and LDS bytes, or a null kernel
// when the arguments need the VALU kernel.  Its workgroups take 32 query
// heads of one KV head (or of a pair) each.  From 3 heads per KV head it
// outruns the VALU kernel (32/8 at d128: 5.70 vs 5.55-5.67 TB/s, 24/8 E4M3
// 4.26-4.35 vs 4.08); at 2 the VALU kernel is as fast or faster.
constexpr int DECODE_GQA_MIN_GROUP = 3;
// Most query rows per request the matrix-core decode takes (its 32 columns
// hold 32 / rows query heads).
constexpr int DECODE_GQA_MAX_ROWS = 16;
struct GqaChoice {
  DecodeKernel kern;
  size_t lds;
  int pack;   // KV heads per workgroup (2: neighbouring 64-dim or 128-dim E4M3 heads, PACK = 2)
};
GqaChoice pick_decode_gqa(const fa_attn_args& a);

}  // namespace fa_decode
