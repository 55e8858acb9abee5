// Split-KV decode on the matrix cores for large GQA groups: one workgroup
// takes up to 32 query heads of one KV head (one query token each) and a
// split of its keys, so every K/V byte read from HBM feeds MFMAs for all of
// them.  The VALU decode kernel (decode_kernel.h) spends per head and key a
// 16-lane dot product and P.V FMAs; with large groups that arithmetic, not
// HBM, sets its pace (Hq/Hkv = 128/8 at d128: 2.3 TB/s, 40/8: 4.5; this
// kernel: 5.2-5.3 and 5.7), and from 3 query heads per KV head this kernel
// is the faster one.  Here the scores of 32 keys x 32 head columns are one
// v_mfma_f32_32x32x16 chain, exactly as in the prefill kernel with the
// group's heads in place of query rows (counterpart of the reference's decode
// route, flash_attn_mps/_decode.py:40-99 and
// kernels/attention_decode.metal:18-149).
//
// * Each of the 4 waves owns the 32-key stages w, w + 4, ... of the split and
//   streams their 16-key groups (global -> LDS DMA, non-temporal: every K/V
//   byte is read once per head tile) through private slots, so the waves
//   never wait on each other inside the loop; at the end they combine (m, l,
//   O) through LDS.  16-bit slots hold one stage (16 KiB at d128, so two
//   workgroups share a CU); each refill is issued as soon as the current
//   stage has read its half (K after S^T, V after P.V), so a wave's loads
//   overlap its own arithmetic.  E4M3 slots hold raw rows only, half the
//   size, so they hold two stages (paired 128-dim E4M3 heads, whose slot
//   rows are two heads long, one).  Rings of 3-5 16-bit slots per wave (one
//   workgroup per CU) measured 4-25% slower at d128 and up to 36% at d64:
//   fewer waves per CU cost more than the prefetch gains.
// * LDS layouts per 16-key slot: K as in the prefill kernel
//   (prefill_kernel.h), rows holding key sigma(r) with 16-byte chunks
//   XOR-swizzled by (r / 2) % 8, 64-dim column groups of 16 rows x 128
//   bytes; 16-bit V in 64-dim column groups of 16 rows x 128 bytes with the
//   64-byte halves of every other row pair swapped, so that each DMA
//   instruction reads whole 128-byte lines and the transposed reads are
//   conflict-free.  S^T = K Q^T (A = K from LDS, B = Q^T in registers), P
//   rounded to the query type, O^T += V^T P^T with V^T read by
//   ds_read_b64_tr_b16.  E4M3: K and V stay raw (rows of D bytes, chunks
//   XOR-swizzled); K operands are widened in registers after 8-byte reads,
//   V^T comes through ds_read_b64_tr_b8 and is widened the same way.
// * Supports 16-bit queries over K/V of their type or E4M3 (with descales),
//   head dims 64 and 128 (Dqk = Dv), outputs of the query's type, packed or
//   paged K/V (page size a multiple of 16), sinks, softcap, windows, 1-16
//   query rows per request; the host keeps other combinations on the VALU
//   kernel.  Neighbouring KV heads (64-dim, or 128-dim E4M3) can run in
//   pairs whose rows the slots hold as one row (PACK below), so that each
//   DMA instruction reads runs of two head rows.
#ifndef FA_DECODE_GQA_H
#define FA_DECODE_GQA_H

#include "decode_kernel.h"
#include "prefill_kernel.h"

namespace fa_decode_gqa {

using namespace fa_prefill;

constexpr int GQA_THREADS = 256;   // 4 waves
constexpr int GQA_HEADS = 32;      // head columns per workgroup (one MFMA tile)
constexpr int GQA_STAGE = 32;      // keys per wave stage
constexpr float GQA_RESCALE = 8.0f;  // log2 headroom before a column's running max moves
#ifndef FA_GQA_NT
#define FA_GQA_NT 1
#endif
constexpr bool GQA_NT = FA_GQA_NT;  // non-temporal K/V DMA

// One 16-key slot: K then V, each D / 64 column groups of 16 rows x 128
// bytes (16-bit) or 16 raw rows of D bytes (E4M3); slots per wave: E4M3
// rings hold two stages, except for paired heads, whose rows are twice as
// long.  D is the row the slots hold (two heads' rows when paired).
template <int D, bool FP8> constexpr int gqa_slot_bytes() { return FP8 ? 32 * D : 64 * D; }
template <int D, bool FP8, int PACK> constexpr int gqa_slots() { return FP8 && PACK == 1 ? 4 : 2; }
template <int D, bool FP8, int PACK> constexpr int gqa_lds_bytes() {
  const int ring = 4 * gqa_slots<D, FP8, PACK>() * gqa_slot_bytes<D, FP8>();
  const int combine = 4 * GQA_HEADS * (D / PACK + 4 + 2) * 4;
  return ring > combine ? ring : combine;
}

// One 8-row block of each of N 64-dim column groups (16 rows x 128 bytes
// apart): one DMA instruction per 8 rows x 128 bytes.
template <int N, int I = 0>
FA_DEV void dma_columns_gqa(__amdgpu_buffer_rsrc_t rsrc, char* lds, int voffset) {
  if constexpr (I < N) {
    dma16<128 * I, GQA_NT>(rsrc, lds + I * 16 * 128, voffset);
    dma_columns_gqa<N, I + 1>(rsrc, lds, voffset);
  }
}

// ds_read_b64_tr_b8: 8 bytes, transposed across the lanes of each 16-lane
// group (see the E4M3 V^T reads below).
FA_DEV u32x2 lds_read_tr8(const char* base, int off) {
  typedef __attribute__((ext_vector_type(2))) int i32x2_t;
  typedef __attribute__((address_space(3))) i32x2_t lds_i32x2;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(base + off)));
}

// s_waitcnt vmcnt(N) (the LDS DMAs of all but the N most recent
// instructions have landed), and s_waitcnt lgkmcnt(0) (this wave's LDS
// reads and writes are done).
template <int N>
FA_DEV void wait_dma_older_than() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
FA_DEV void wait_lds() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }
// s_waitcnt vmcnt(n * PER) for a runtime n in [0, MAXN].
template <int PER, int MAXN>
FA_DEV void wait_dma_groups(int n) {
  if constexpr (MAXN == 0) {
    wait_dma_older_than<0>();
  } else {
    if (n >= MAXN) wait_dma_older_than<MAXN * PER>();
    else wait_dma_groups<PER, MAXN - 1>(n);
  }
}

// KT: K/V storage type, T or E4M3.  E4M3 slots hold the raw K rows (16 rows
// x D bytes, rows at sigma(r), 16-byte chunks XOR-swizzled) and the raw V
// rows (16 x D bytes, chunks XOR-swizzled): K operands widen in registers
// after an 8-byte LDS read, V^T comes through ds_read_b64_tr_b8 and widens in
// registers the same way, and the descales scale the scores and the output.
// PACK = 2: two neighbouring KV heads of DH = D / 2 dims, stored next to
// each other in every key row, run in one workgroup whose slots hold both
// heads' rows as one row of D elements, so each DMA instruction reads runs
// of 2 x DH elements (64-dim heads: 128 bytes of E4M3 or 256 of 16-bit
// instead of 64 / 128; 128-dim E4M3 heads: 256 bytes instead of 128).  The
// workgroup's query heads are the two heads' groups.  S^T = K Q^T runs over
// the whole row with each column's query entering only the k-steps of its
// own head's half (zeros in the other's), so each column gets its own KV
// head's scores; P.V runs over both halves of V into the same DH-dim O^T,
// with each column's probabilities zeroed for the other head's half, so
// every column accumulates only its own head's values.  Descales are per
// column (its KV head).
template <typename T, int D, bool CAP, typename KT = T, int PACK = 1>
__global__ __launch_bounds__(GQA_THREADS, 1) void decode_gqa_kernel(const fa_attn_args a, const int span) {
  static_assert(D == 64 || D == 128 || D == 256, "rows of 64, 128 or 256 elements");
  static_assert((PACK == 1 && D <= 128) || (PACK == 2 && (D == 128 || (D == 256 && KT::id == FA_E4M3))),
                "paired heads: 64-dim heads, or 128-dim E4M3 heads");
  constexpr int DH = D / PACK;            // the heads' own dims
  constexpr bool FP8 = KT::id == FA_E4M3;
  constexpr int EB = KT::bytes;           // bytes per K/V element
  constexpr int KSTEPS = D / 16;          // k-steps of S^T = K Q^T over a slot row
  constexpr int KPH = KSTEPS / PACK;      // k-steps per head
  constexpr int KG = D / 64;              // 64-dim column groups of a K slot
  constexpr int DB = D / 32;              // 32-dim blocks of V^T in a slot row
  constexpr int DBH = DH / 32;            // 32-dim blocks of O^T (one head)
  constexpr int KGROUP = 16 * 128;        // one column group: 16 rows x 128 bytes
  constexpr int KBYTES = KG * KGROUP, SLOT = gqa_slot_bytes<D, FP8>(), NSLOT = gqa_slots<D, FP8, PACK>();
  static_assert(NSLOT >= 2, "a stage's two slots");
  constexpr bool RING2 = NSLOT == 4;      // slots hold two stages (E4M3, unpaired)

  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  char* const ring = smem + wave * NSLOT * SLOT;   // this wave's slots

  // Columns: ntok = max_seqlen_q query rows (tokens) per request, nh =
  // 32 / ntok query heads per workgroup; column c is head h0 + c / ntok,
  // token c % ntok (one token: column c = head h0 + c).  A request's tokens
  // are its last q_len key positions.
  // Grid: x = (virtual) KV head * head tiles + tile, y = split, z = request.
  // Virtual KV head kh holds KV heads PACK kh .. PACK kh + PACK - 1 and their
  // PACK * gr query heads, numbered contiguously.
  const int ntok = a.max_seqlen_q > 1 ? (int)a.max_seqlen_q : 1, nh = GQA_HEADS / ntok;
  const int gr = (int)(a.heads_q / a.heads_k);   // query heads per KV head
  const int group = PACK * gr;
  const int tiles = (group + nh - 1) / nh;
  const int kh = blockIdx.x / tiles, t0 = (blockIdx.x % tiles) * nh;
  const int nheads = min(nh, group - t0);
  const int h0 = kh * group + t0;
  const int S = a.num_splits;
  const fa_decode::SplitItem item = fa_decode::split_item(a, ntok, span);
  if (!item.ok) return;
  const int split = item.split;
  const int64_t b = item.b;
  const RequestInfo r = item.r;
  const int vis_begin = fa_decode::decode_vis_begin(a, r.k_len, r.q_len);
  const int begin = vis_begin + split * span;
  const int end = min(r.k_len, begin + span);
  if (split > 0 && begin >= end) return;
  // This lane's column.
  const int chead = l32 / ntok, ctok = l32 - chead * ntok;
  const bool col_ok = chead < nheads && ctok < r.q_len;
  // KV head of query head h0 + c (c < nheads), as its part of the virtual
  // head; columns past the group take the last part (they hold no query).
  auto part_of = [&](int c) { return PACK > 1 ? min((h0 + c) / gr - PACK * kh, PACK - 1) : 0; };
  const int cpart = part_of(chead);

  // Zeroed V buffers: rows the DMA does not write (past the request) then
  // hold finite values, which a zero probability keeps out of O.  The
  // stores land before this wave's first DMA is issued.
  for (int i = lane; i < NSLOT * SLOT / 16; i += 64) {
    const int off = 16 * i;
    if ((off % SLOT) >= (FP8 ? 16 * D : KBYTES)) *(u32x4*)(ring + off) = u32x4{0u, 0u, 0u, 0u};
  }
  wait_lds();

  // Q^T operands: k-step kk of a head, lane (l32, hh) holds its column's
  // query (token ctok, head h0 + chead), dims 16 kk + 8 hh .. +8 (zeros for
  // columns past the group or the request's tokens).
  u32x4 qop[KPH];
  {
    const uint16_t* qp = (const uint16_t*)a.q + (int64_t)(r.q_begin + (col_ok ? ctok : 0)) * a.q_stride[0] +
                         (int64_t)(h0 + (col_ok ? chead : 0)) * a.q_stride[1] + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < KPH; ++kk) qop[kk] = col_ok ? *(const u32x4*)(qp + 16 * kk) : u32x4{0u, 0u, 0u, 0u};
  }

  // Descales of this column's KV head (one per workgroup unless packed).
  const int ckh = PACK * kh + cpart;
  const float kdsc = descale_of(a.q_descale, a.q_descale_stride, b, ckh) * descale_of(a.k_descale, a.k_descale_stride, b, ckh);
  const float c_scale = a.softmax_scale * kdsc * LOG2E;   // raw dot -> log2 units
  const float cap_in = CAP ? 2.0f * LOG2E * a.softmax_scale * kdsc / a.softcap : 0.0f;
  const float cap_out = a.softcap * LOG2E;
  // A sink logit seeds the state of one wave of split 0 (max = sink, sum = 1).
  const bool seed = a.sinks && split == 0 && wave == 0;
  float m_run = seed && col_ok ? a.sinks[(int64_t)(h0 + chead) * a.sink_stride] * LOG2E : -INFINITY;
  float l_run = seed && hh == 0 ? 1.0f : 0.0f;
  f32x16 o[DBH];
#pragma unroll
  for (int db = 0; db < DBH; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;

  // ---- DMA.  Storage position of key j: k_base + left + j (a packed row,
  // or slot j of the request's pages).  Stages cover 32 storage positions
  // aligned to 32; a stage is two 16-key groups, each inside one page (the
  // host requires a page size that is a multiple of 16).  K: one instruction
  // moves one 8-row block of one column group (lane p -> LDS row 8 rb + p / 8,
  // slot p % 8 holding chunk (p % 8) ^ ((row / 2) % 8); row r holds key
  // sigma(r) of its group); V likewise, unswizzled and unpermuted (lane p ->
  // row 8 rb + p / 8, chunk p % 8).
  const int P = (int)a.page_size;
  const int pos_lo = r.k_base + r.left + begin, pos_hi = r.k_base + r.left + end;   // this split's keys
  // Keys this lane's column sees, as storage positions [col_lo, col_hi):
  // the split's, clipped to the token's window (left: position - WL; right:
  // the position itself when causal, + WR with a right window); none for
  // columns without a query.
  int col_lo = INT_MAX, col_hi = INT_MIN;
  if (col_ok) {
    const int qpos = r.k_len - r.q_len + ctok;
    int hi = r.k_len;
    if (r.causal) hi = qpos + 1;
    else if (a.window_right >= 0) hi = min(hi, qpos + a.window_right + 1);
    const int lo = a.window_left >= 0 ? max(qpos - a.window_left, 0) : 0;
    col_lo = max(pos_lo, r.k_base + r.left + lo);
    col_hi = min(pos_hi, r.k_base + r.left + hi);
  }
  const int pos_end = r.k_base + r.left + r.k_len;                                   // the request's end
  const uint32_t krow_b = (uint32_t)(EB * a.k_stride[1]), vrow_b = (uint32_t)(EB * a.v_stride[1]);
  const uint32_t kpage_b = (uint32_t)(EB * a.k_stride[0]), vpage_b = (uint32_t)(EB * a.v_stride[0]);
  const char* const khead = (const char*)a.k + EB * (int64_t)(PACK * kh) * a.k_stride[2];
  const char* const vhead = (const char*)a.v + EB * (int64_t)(PACK * kh) * a.v_stride[2];
  const int32_t* const trow = P ? a.block_table + b * a.bt_stride[0] : nullptr;
  int kdoff[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int drow = 8 * rb + (lane >> 3);   // row within the 16-key group
    kdoff[rb] = (int)(sigma(drow) * krow_b) + (((lane & 7) ^ ((drow >> 1) & 7)) * 16);
  }
  // V rows (16-bit, 128 bytes): 16-byte chunk j of row r at position j ^
  // vswz(r), which swaps the row's 64-byte halves on rows with bit 1 set, so
  // the four rows {t, t + 1, t + 2, t + 3} (t = 0, 4, 8, 12) that one half
  // of a transposed read touches fall on the four distinct 64-byte bank
  // quarters (unswizzled 128-byte rows put two of them on the same quarter).
  auto vswz = [](int row) { return 4 * ((row >> 1) & 1); };
  int vdoff[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int row = 8 * rb + (lane >> 3);
    vdoff[rb] = (int)(row * vrow_b) + (((lane & 7) ^ vswz(row)) * 16);
  }
  // E4M3 rows of D bytes: one instruction moves 1024 / D rows (lane p -> row
  // 1024 / D * ib + p / NCH, 16-byte position p % NCH of NCH = D / 16); K
  // rows hold key sigma(row) and position q holds chunk q ^ swz8(row), which
  // spreads the 8-byte K operand reads of 16 rows over distinct bank slots.
  constexpr int NCH = D / 16;
  auto swz8 = [](int row) { return D == 256 ? row & 15 : D == 128 ? (row >> 1) & 7 : (row >> 2) & 3; };
  // Raw E4M3 V rows: 16-byte chunk q at position q ^ vswz8(row), so the 16
  // lanes of one transposed read (8 rows x two 8-byte halves of one chunk)
  // fall on 16 distinct bank pairs.
  auto vswz8 = [](int row) { return D >= 128 ? row & 7 : (row >> 2) & 3; };
  int kdoff8[KG], vdoff8[KG];
#pragma unroll
  for (int ib = 0; ib < KG; ++ib) {
    const int row = (1024 / D) * ib + lane / NCH, q = lane % NCH;
    kdoff8[ib] = (int)(sigma(row) * krow_b) + ((q ^ swz8(row)) * 16);
    vdoff8[ib] = (int)(row * vrow_b) + ((q ^ vswz8(row)) * 16);
  }
  // Buffer descriptor of the 16-key group at storage position pos (a
  // multiple of 16), covering only its keys in [pos_lo, pos_end): the base is
  // the row of the first such key (row `first` of the group) and the size
  // ends at the request's last key.  Lanes address their row relative to
  // that base (voffset - first * row_b), so rows before pos_lo get negative,
  // i.e. out-of-range offsets and are never read (they may be left padding
  // holding anything); rows past the request are out of range at the top.
  // Stage i of this wave: storage positions st_pos(i) .. +32, its 16-key
  // groups 2 i and 2 i + 1; group j lives in slot j % NSLOT.
  const int pos0 = pos_lo & ~(GQA_STAGE - 1);
  auto st_pos = [&](int i) { return pos0 + GQA_STAGE * (wave + 4 * i); };
  const int nst = pos_hi > pos0 + GQA_STAGE * wave ? (pos_hi - pos0 - GQA_STAGE * wave + 4 * GQA_STAGE - 1) / (4 * GQA_STAGE) : 0;
  const int ngroups = 2 * nst;
  auto group_pos = [&](int j) { return st_pos(j >> 1) + 16 * (j & 1); };
  // Pages of this wave's groups, 64 at a time: lane l of `pages` holds the
  // block-table entry of group 64 chunk + l (0 for groups with no key of the
  // split), read once per chunk with one vector load; each group then takes
  // its entry with v_readlane instead of a scalar load and its wait.  The
  // load is waited for with vmcnt(0): free for the first chunk (before any
  // DMA); a wave with more than 64 groups (over 4096 keys per workgroup, e.g.
  // one split per request on long contexts) reloads mid-loop, where that
  // wait also drains the DMAs of the stages it already has in flight, once
  // per 32 of its stages.
  int chunk = -1;
  uint32_t pages = 0;
  auto page_of_group = [&](int j) {
    if ((j >> 6) != chunk) {
      chunk = j >> 6;
      const int jj = 64 * chunk + lane, pos = group_pos(jj);
      const bool need = jj < ngroups && pos + 16 > pos_lo && pos < pos_end;
      pages = need ? (uint32_t)trow[(int64_t)(pos / P) * a.bt_stride[1]] : 0u;
      wait_dma_older_than<0>();
    }
    return (uint32_t)__builtin_amdgcn_readlane((int)pages, j & 63);
  };
  auto group_rsrc = [&](const char* head, uint32_t row_b, uint32_t page_b, int j, int row_bytes, int& shift) {
    const int pos = group_pos(j);
    const int first = min(max(pos_lo - pos, 0), 16);
    const int nvalid = min(max(pos_end - pos, 0), 16) - first;
    const char* g = head;
    if (nvalid > 0) {
      if (P) {
        const uint32_t blk = page_of_group(j);
        g = head + (uint64_t)blk * page_b + (uint64_t)(uint32_t)(pos % P + first) * row_b;
      } else {
        g = head + (uint64_t)(uint32_t)(pos + first) * row_b;
      }
    }
    shift = __builtin_amdgcn_readfirstlane(first * (int)row_b);
    const int bytes = __builtin_amdgcn_readfirstlane(nvalid > 0 ? (nvalid - 1) * (int)row_b + row_bytes : 0);
    // The base is wave-uniform; readfirstlane states it, so the descriptor
    // stays in scalar registers as the DMA instruction requires.
    const uint64_t gi = (uint64_t)(uintptr_t)g;
    const uint64_t gu = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(gi >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)gi);
    return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)gu, (short)0, bytes, 0x00020000);
  };
  // Slot of group c of stage i: 16-bit K and V, or paired E4M3 rows, of one
  // stage (slots 0, 1); unpaired E4M3 raw K and V rows of two stages (slots
  // 2 (i % 2) + c).
  auto slot_of = [&](int i, int c) -> char* { return ring + (RING2 ? 2 * (i & 1) + c : c) * SLOT; };
  // DMA instructions per stage (two groups): 4 KG each for 16-bit K and V,
  // 2 KG each for E4M3 K and V.
  constexpr int KD = FP8 ? 2 * KG : 4 * KG, VD = KD;
  auto dma_k_stage = [&](int i) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      char* const kb = slot_of(i, c);
      int kshift;
      const auto kr = group_rsrc(khead, krow_b, kpage_b, 2 * i + c, EB * D, kshift);
      if constexpr (FP8) {
#pragma unroll
        for (int ib = 0; ib < KG; ++ib) dma16<0, GQA_NT>(kr, kb + 1024 * ib, kdoff8[ib] - kshift);
      } else {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) dma_columns_gqa<KG>(kr, kb + 8 * rb * 128, kdoff[rb] - kshift);
      }
    }
  };
  auto dma_v_stage = [&](int i) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      char* const kb = slot_of(i, c);
      int vshift;
      const auto vr = group_rsrc(vhead, vrow_b, vpage_b, 2 * i + c, EB * D, vshift);
      if constexpr (FP8) {
#pragma unroll
        for (int ib = 0; ib < KG; ++ib) dma16<0, GQA_NT>(vr, kb + 16 * D + 1024 * ib, vdoff8[ib] - vshift);
      } else {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) dma_columns_gqa<KG>(vr, kb + KBYTES + 8 * rb * 128, vdoff[rb] - vshift);
      }
    }
  };

  // Operand read offsets (bytes within a slot): K (A of S^T) row l32 % 16 of
  // the stage's slot l32 / 16, chunk 2 (kk % 4) + hh of column group kk / 4;
  // V^T through ds_read_b64_tr_b16 with the prefill kernel's lane pattern
  // (16-lane group g, lane a + 4 t': row 8 (g / 2) + t' (+ 4 for the second
  // read), dims 16 (g % 2) + 4 a of 32-dim block db, which is half db % 2 of
  // column group db / 2), keys 16 c .. +16 from the stage's slot c.
  const int r16 = l32 & 15;
  int krd[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) krd[s] = r16 * 128 + (((2 * s + hh) ^ ((r16 >> 1) & 7)) * 16);
  const int vg16 = lane >> 4, vi = lane & 15, va = vi & 3, vt = vi >> 2;
  const int vrow = 8 * (vg16 >> 1) + vt;   // (+ 4 for the second read: same swizzle)
  const int vrd0 = KBYTES + vrow * 128 + 64 * (vswz(vrow) >> 2) + (4 * (vg16 & 1) + va) * 8;   // even blocks
  const int vrd1 = vrd0 + 64 - 128 * (vswz(vrow) >> 2);                                        // odd blocks
  // E4M3: K operand k-step kk = 8 bytes of raw row r16 (dims 16 kk + 8 hh
  // .. +8, chunk kk at position kk ^ swz8(r16)).
  int krd8[FP8 ? KSTEPS : 1];
#pragma unroll
  for (int kk = 0; kk < (FP8 ? KSTEPS : 1); ++kk) krd8[kk] = r16 * D + ((kk ^ swz8(r16)) * 16) + 8 * hh;
  // E4M3 V^T straight from the raw rows through ds_read_b64_tr_b8, widened in
  // registers: in each 16-lane group g the hardware hands lane i byte i % 8
  // of the 8 bytes read by lanes i / 8, i / 8 + 2, ..., i / 8 + 14, in that
  // order.  Lane s of group g reads row 8 (g / 2) + s / 2, dims 32 db + 16
  // (g % 2) + 8 (s % 2) .. +8, so lane 16 g + i receives dim 32 db + 16 (g %
  // 2) + i of keys 8 (g / 2) .. +8: the A operand of O^T += V^T P^T.
  const int v8row = 8 * (vg16 >> 1) + (vi >> 1);
  int vrd8[FP8 ? DB : 1];
#pragma unroll
  for (int db = 0; db < (FP8 ? DB : 1); ++db)
    vrd8[db] = 16 * D + v8row * D + (((2 * db + (vg16 & 1)) ^ vswz8(v8row)) * 16) + 8 * (vi & 1);

  // Stage i.  K(i) landed (V(i) may still be in flight) -> S^T -> the next
  // K DMA into the K halves just read -> softmax -> V(i) landed -> P.V ->
  // the next V DMA into the V halves just read.  One-stage rings (16-bit,
  // paired E4M3) refill with stage i + 1; two-stage rings (unpaired E4M3)
  // with stage i + 2 while stage i + 1 is already in flight.  Each load
  // overlaps the wave's own arithmetic instead of following it.
  auto stage = [&](int i, bool more) {
    char* const slot0 = slot_of(i, 0);
    char* const slot1 = slot_of(i, 1);
    // K(i) landed; newer: V(i), and with two-stage rings also stage i + 1.
    if (RING2 && more) wait_dma_older_than<2 * VD + KD>();
    else wait_dma_older_than<VD>();
    const char* const kb = l32 < 16 ? slot0 : slot1;
    // Paired: a column's query enters only the k-steps of its own head's
    // half of the slot rows (zeros in the other half's).
    f32x16 s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.0f;
    // All ones for the first head's columns; opaque per stage, so that the
    // masked query copies are formed at their use, not kept for the loop.
    uint32_t first = cpart == 0 ? ~0u : 0u;
    asm volatile("" : "+v"(first));
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      u32x4 av;
      if constexpr (FP8) {
        const u32x2 w = *(const u32x2*)(kb + krd8[kk]);
        av = u32x4{widen_fp8_pair<T, false>(w[0]), widen_fp8_pair<T, true>(w[0]), widen_fp8_pair<T, false>(w[1]),
                   widen_fp8_pair<T, true>(w[1])};
      } else {
        av = lds_read16(kb, krd[kk % 4] + (kk / 4) * KGROUP);
      }
      u32x4 qv = qop[kk % KPH];
      if constexpr (PACK > 1) {
        const uint32_t keep = kk < KPH ? first : ~first;
#pragma unroll
        for (int e = 0; e < 4; ++e) qv[e] &= keep;
      }
      s = mfma32<T>(av, qv, s);
    }
    wait_lds();   // K reads of stage i done
    if constexpr (RING2) {
      if (i + 2 < nst) dma_k_stage(i + 2);
    } else {
      if (more) dma_k_stage(i + 1);
    }
    // s[e] = score of storage position st_pos(i) + 16 (e >> 3) + 8 hh + (e & 7).
    const int p0 = st_pos(i) + 8 * hh;
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float v = s[e];
      if constexpr (CAP) v = cap_out * (1.0f - 2.0f * __builtin_amdgcn_rcpf(fast_exp2(cap_in * v) + 1.0f));
      else v *= c_scale;
      const int pos = p0 + 16 * (e >> 3) + (e & 7);
      v = (pos >= col_lo && pos < col_hi) ? v : -INFINITY;
      s[e] = v;
      mx = fmaxf(mx, v);
    }
    mx = max_hh(mx);
    // Lazy rescale: the running max moves only when a score passes it by
    // more than GQA_RESCALE (log2 units; always for the first finite max),
    // so probabilities stay <= 2^GQA_RESCALE and O is rescaled in few
    // stages even when 32 columns each raise their max now and then.
    const bool need = mx > m_run + GQA_RESCALE;
    const float m_new = need ? mx : m_run;
    const float mref = m_new == -INFINITY ? 0.0f : m_new;
    const float f = need ? fast_exp2((m_run == -INFINITY ? mref : m_run) - mref) : 1.0f;
    m_run = m_new;
    l_run *= f;
    if (__builtin_expect(__any(f != 1.0f), 0)) {
#pragma unroll
      for (int db = 0; db < DBH; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[db][e] *= f;
    }
    float psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float p = fast_exp2(s[e] - mref);
      s[e] = p;
      psum += p;
    }
    l_run += psum;
    // P^T operands per head half: a column's probabilities for its own
    // head's half of the V rows, zeros for the other half.
    u32x4 pop[PACK][2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t w = pack2<T>(s[8 * c + 2 * q], s[8 * c + 2 * q + 1]);
#pragma unroll
        for (int u = 0; u < PACK; ++u) pop[u][c][q] = PACK == 1 || cpart == u ? w : 0u;
      }
    // V(i) landed; newer: K(i + 1) with one-stage rings; stage i + 1 and
    // K(i + 2) with two-stage rings.
    if constexpr (RING2) {
      if (i + 2 < nst) wait_dma_older_than<2 * KD + VD>();
      else if (more) wait_dma_older_than<KD + VD>();
      else wait_dma_older_than<0>();
    } else {
      if (more) wait_dma_older_than<KD>();
      else wait_dma_older_than<0>();
    }
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const char* const vb = c ? slot1 : slot0;
        u32x4 av;
        if constexpr (FP8) {
          const u32x2 w = lds_read_tr8(vb, vrd8[db]);
          av = u32x4{widen_fp8_pair<T, false>(w[0]), widen_fp8_pair<T, true>(w[0]), widen_fp8_pair<T, false>(w[1]),
                     widen_fp8_pair<T, true>(w[1])};
        } else {
          const int vrd = ((db & 1) ? vrd1 : vrd0) + (db >> 1) * KGROUP;
          const u32x2 lo = lds_read_tr(vb, vrd);
          const u32x2 hi = lds_read_tr(vb, vrd + 4 * 128);
          av = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
        o[db % DBH] = mfma32<T>(av, pop[db / DBH][c], o[db % DBH]);
      }
    wait_lds();   // V reads of stage i done
    if constexpr (RING2) {
      if (i + 2 < nst) dma_v_stage(i + 2);
    } else {
      if (more) dma_v_stage(i + 1);
    }
  };

  if (nst > 0) {
    dma_k_stage(0);
    dma_v_stage(0);
  }
  if (RING2 && nst > 1) {
    dma_k_stage(1);
    dma_v_stage(1);
  }
  for (int i = 0; i < nst; ++i) stage(i, i + 1 < nst);

  // ---- Combine the four waves: per head m (log2 units), l and O^T through
  // LDS (the stage buffers are done once every wave passes the barrier).
  const float lt = sum_hh(l_run);
  __syncthreads();
  float* const cm = (float*)smem;                      // [4][32]
  float* const cl = cm + 4 * GQA_HEADS;                // [4][32]
  // [4][32][DH + 4]: the 4-float pad puts the 32 head columns' 16-byte
  // stores of one instruction on distinct bank groups.
  constexpr int CO_ROW = DH + 4;
  float* const co = cl + 4 * GQA_HEADS;
  if (hh == 0) {
    cm[wave * GQA_HEADS + l32] = m_run;
    cl[wave * GQA_HEADS + l32] = lt;
  }
  // o[db][4 g + j] = O^T[dim 32 db + 8 g + 4 hh + j][head l32].
#pragma unroll
  for (int db = 0; db < DBH; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *(float4*)(co + ((int64_t)wave * GQA_HEADS + l32) * CO_ROW + 32 * db + 8 * g + 4 * hh) =
          float4{o[db][4 * g], o[db][4 * g + 1], o[db][4 * g + 2], o[db][4 * g + 3]};
  __syncthreads();
  // Per column, once: the combined max, the four waves' weights times the
  // output scale (written over cm) and the LSE (over cl's first row).  Each
  // column belongs to one thread here, which reads all its entries before
  // writing them.
  const int ncol = nh * ntok;   // <= GQA_HEADS
  if (tid < ncol) {
    float M = cm[tid];
#pragma unroll
    for (int w = 1; w < 4; ++w) M = fmaxf(M, cm[w * GQA_HEADS + tid]);
    const float ref = M == -INFINITY ? 0.0f : M;
    float fw[4], L = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      fw[w] = fast_exp2(cm[w * GQA_HEADS + tid] - ref);
      L += cl[w * GQA_HEADS + tid] * fw[w];
    }
    const float vdsc = descale_of(a.v_descale, a.v_descale_stride, b, PACK * kh + part_of(tid / ntok));
    const float norm = L > 0.0f ? vdsc / L : 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) cm[w * GQA_HEADS + tid] = fw[w] * norm;
    cl[tid] = L > 0.0f ? M * LN2 + logf(L) : -INFINITY;
  }
  __syncthreads();
  // hc / ntok for hc < 32 and 1 <= ntok <= 16 as a multiply by
  // ceil(2^32 / ntok) and a shift (the rounding error stays below 32 / 2^32).
  const uint64_t ntok_inv = ((1ull << 32) + (uint64_t)ntok - 1) / (uint64_t)ntok;
  for (int idx = tid; idx < ncol * DH; idx += GQA_THREADS) {
    const int hc = idx / DH, d = idx - hc * DH;   // column hc: head h0 + hc / ntok, token hc % ntok
    const int th = (int)(((uint64_t)hc * ntok_inv) >> 32), tt = hc - th * ntok;
    if (th >= nheads || tt >= r.q_len) continue;
    float O = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) O += co[((int64_t)w * GQA_HEADS + hc) * CO_ROW + d] * cm[w * GQA_HEADS + hc];
    const int h = h0 + th;
    const int64_t tq = r.q_begin + tt;
    if (S == 1) {
      store_any(a.out, tq * a.out_stride[0] + (int64_t)h * a.out_stride[1] + (int64_t)d * a.out_stride[2], a.out_dtype, O);
      if (d == 0) a.lse[(int64_t)h * a.lse_stride[0] + tq * a.lse_stride[1]] = cl[hc];
    } else {
      // Partial outputs [batch][S][ntok][Hq][D], LSEs [batch][ntok][Hq][S].
      // A workgroup's outputs are ntok runs of 4 D nheads bytes, and the
      // workgroups running together (neighbouring heads and splits of one
      // request) fill neighbouring runs; streaming stores keep the partials
      // from displacing K/V in the caches.  Interleaved 4 D-byte rows (the
      // splits of one row together) cost config 3's speculative step ~6%.
      const int64_t orow = ((b * S + split) * ntok + tt) * a.heads_q + h;
      __builtin_nontemporal_store(O, &a.partial_out[orow * DH + d]);
      if (d == 0) a.partial_lse[((b * ntok + tt) * a.heads_q + h) * S + split] = cl[hc];
    }
  }
}

}  // namespace fa_decode_gqa

#endif  // FA_DECODE_GQA_H
