// MFMA FlashAttention prefill for gfx950 (bf16 / fp16).
//
// Semantics follow the reference's fast path (flash_attn_mps/_attention.py:149-158,
// flash_attn_mps/kernels/attention_fast.metal:103-597) plus the DIFFKV head
// dims and attention sinks of its tiled path (flash_attn_mps/kernels/
// attention.metal:60-181): packed or paged K/V, GQA, lower-right causality,
// optional softcap, left/right sliding windows, a per-head sink logit that joins the softmax
// denominator only, fp32 softmax and natural-log LSE.  Head dims (Dqk, Dv)
// in {(32,32), (64,64), (72,72), (80,80), (96,96), (128,128), (256,256),
// (192,128)}; 32 and 72/80/96 run zero-padded in the 64 and 128 tiles.
//
// gfx950 design
// * A workgroup is W waves; each wave owns 32 query rows of one head.  K/V
//   tiles of 64 keys live in LDS, two K and two V buffers.
// * Tiles move global -> LDS with buffer_load ... lds (16 bytes a lane, one
//   contiguous KiB per instruction): no registers, no VALU.  Every 16-key
//   group gets a scalar buffer descriptor bounded at the request's last key,
//   so rows past the end read as zero; lane offsets are loop-invariant.
// * LDS layout.  K: 64-dim column groups of 64 rows x 128 bytes, the eight
//   16-byte chunks of a row XOR-swizzled by (row / 2) % 8.  V: 32-dim blocks
//   of 64 rows x 64 bytes, unswizzled: the eight rows {0..3, 8..11} (+4k)
//   that one transpose read touches then cover the banks evenly.  Every
//   operand read is bank-conflict free and addressed as a lane register plus
//   an immediate.
// * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16 (A =
//   K rows from LDS, B = Q^T held in registers for the whole kernel).  A lane
//   holds 32 keys of ONE query column, so the row max / sum are in-lane plus
//   one v_permlane32_swap.  K rows are stored at sigma(r) (bits 2 and 3 of r
//   swapped) so each lane's 8 consecutive accumulators are 8 consecutive
//   keys: rounded to bf16/fp16 they are directly the B operand of
//   O^T += V^T P^T.  The V^T operand is read from the row-major V tile with
//   ds_read_b64_tr_b16 (two per MFMA).
// * Software pipeline per wave over 32-key stages: while the MFMAs of
//   S(s+1) = K(s+1) Q^T run, the VALU turns S(s) into P(s) (exp2, pack, row
//   sums); while the MFMAs of O += V(s) P(s) run, the VALU takes the row max
//   of S(s+1).  One barrier per 64-key tile; the next tiles' K and V are in
//   flight meanwhile.
// * exp2 with softmax_scale*log2(e) folded into one FMA; the running max only
//   moves (and O is rescaled) when a tile raises it by more than 2^8.
// * Work is ordered per XCD: each XCD runs whole (request, KV head) pairs one
//   after another, query blocks heaviest-first within a pair, so resident
//   workgroups share K/V in their XCD's L2.
#ifndef FA_PREFILL_KERNEL_H
#define FA_PREFILL_KERNEL_H

#include "attn_common.h"

#include <climits>
#include <type_traits>

namespace fa_prefill {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr float PF_RESCALE = 8.0f;        // log2 headroom before the running max moves
constexpr int PF_BN = 64;                 // keys per tile
constexpr int PF_GROUP_BYTES = 64 * 128;  // one 64-dim column group of a K tile
constexpr int PF_VBLOCK_BYTES = 64 * 64;
// K/V load modes of the main loop (see dma_k / dma_v).
constexpr int PF_ANY_TILE = 0, PF_FULL_PACKED = 1, PF_FULL_PAGED = 2;  // one 32-dim block of a V tile

template <typename T> FA_DEV f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);
template <> FA_DEV f32x16 mfma32<BF16T>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <> FA_DEV f32x16 mfma32<F16T>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

typedef __attribute__((ext_vector_type(8))) int i32x8;

// S += A B over 64 E4M3 dims with v_mfma_f32_32x32x64_f8f6f4 (no block
// scales).  Lane (r, h) holds 32 bytes of row r; the instruction contracts
// over (lane half, byte), so A and B need only split each 64-dim step the
// same way: here lane half h holds dims 32 h .. 32 h + 31 in byte order.
// E4M3 x E4M3 products are exact in fp32.
FA_DEV f32x16 mfma32_fp8(i32x8 a, i32x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// Two fp32 values -> one word of two 16-bit values (RNE).
template <typename T> FA_DEV uint32_t pack2(float lo, float hi);
template <> FA_DEV uint32_t pack2<BF16T>(float lo, float hi) {
  bf16x2 v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}
template <> FA_DEV uint32_t pack2<F16T>(float lo, float hi) {
  f16x2 v;
  v[0] = (_Float16)lo;
  v[1] = (_Float16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// Two E4M3 codes (bytes 2 HI .. 2 HI + 1 of w) -> two T values, exactly.
template <typename T, bool HI> FA_DEV uint32_t widen_fp8_pair(uint32_t w);
template <> FA_DEV uint32_t widen_fp8_pair<BF16T, false>(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
}
template <> FA_DEV uint32_t widen_fp8_pair<BF16T, true>(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
}
template <> FA_DEV uint32_t widen_fp8_pair<F16T, false>(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
}
template <> FA_DEV uint32_t widen_fp8_pair<F16T, true>(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
}
// w with its two 8-byte halves exchanged when `swap` (one select per dword).
FA_DEV u32x4 halves_swapped_if(u32x4 w, int swap) {
  return swap ? u32x4{w[2], w[3], w[0], w[1]} : w;
}

// 16 E4M3 codes -> 16 T values (dims 0..7 in lo, 8..15 in hi).
template <typename T>
FA_DEV void widen_fp8_16(u32x4 w, u32x4& lo, u32x4& hi) {
  lo = u32x4{widen_fp8_pair<T, false>(w[0]), widen_fp8_pair<T, true>(w[0]), widen_fp8_pair<T, false>(w[1]),
             widen_fp8_pair<T, true>(w[1])};
  hi = u32x4{widen_fp8_pair<T, false>(w[2]), widen_fp8_pair<T, true>(w[2]), widen_fp8_pair<T, false>(w[3]),
             widen_fp8_pair<T, true>(w[3])};
}

// Swap bits 2 and 3 of a row index (an involution).
FA_DEV int sigma(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

// LDS bank slots on gfx950, measured with probe kernels
// (SQ_LDS_BANK_CONFLICT): a 16-byte read is served 16 consecutive lanes a
// cycle, each lane's slot being address bits [7:4] XOR (bits [9:8] << 1); a
// 16-byte write is served 8 consecutive lanes a cycle, slot = bits [6:4].
// The FP8 staging rows are stored with their 16-byte chunks permuted (chunk
// u of row r at u ^ stage_rows(r), inside the row) so that the widening
// passes, which read 4 consecutive keys x 4 consecutive chunks per 16-lane
// group, hit 16 distinct read slots.
template <int D> FA_DEV int stage_rows(int r) {
  if constexpr (D == 128) return 4 * ((r >> 1) & 1);
  else if constexpr (D == 256) return 4 * (r & 3);
  else return 0;
}

// x combined with the value of lane ^ 32 (v_permlane32_swap exchanges the
// wave halves; max / sum of the two results is symmetric in them).
FA_DEV float max_hh(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
FA_DEV float sum_hh(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 16 bytes a lane from a buffer straight into LDS at lds + 16 * lane
// (buffer_load_dwordx4 ... lds: LDS address = m0 + IMM + 16 * lane, global
// address = base + voffset + IMM).  Written as inline assembly so that the
// compiler does not track it: it treats an LDS-DMA load as a possible writer
// of whatever a later ds_read_b64_tr_b16 reads and puts an
// `s_waitcnt vmcnt(0)` before the first transposed V read after it, which
// stalled every wave in each tile until the DMAs it had just issued for the
// NEXT tiles had landed.  The kernel orders DMA writes and LDS reads itself
// (s_waitcnt vmcnt(0) + barrier at each tile start, and DMAs only ever
// target buffers no wave reads until then).  m0 (a register the compiler
// reserves, so it cannot be declared clobbered) is saved and restored
// around the load, with the one wait state the hardware needs between
// writing m0 and the load.  NT marks the load non-temporal (streamed data
// read once, as in decode).
template <int IMM, bool NT = false>
FA_DEV void dma16(__amdgpu_buffer_rsrc_t rsrc, char* lds, int voffset) {
#if __HIP_DEVICE_COMPILE__
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)(lds - IMM));
  uint32_t saved;
  if constexpr (NT) {
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen offset:%4 nt lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(base), "v"(voffset), "s"(rsrc), "i"(IMM)
        : "memory");
  } else {
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen offset:%4 lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(base), "v"(voffset), "s"(rsrc), "i"(IMM)
        : "memory");
  }
#endif
}

// One row block (8 rows x 128 bytes) of each of N column groups.
template <int N, int I = 0>
FA_DEV void dma_columns(__amdgpu_buffer_rsrc_t rsrc, char* lds, int voffset) {
  if constexpr (I < N) {
    dma16<128 * I>(rsrc, lds + I * PF_GROUP_BYTES, voffset);
    dma_columns<N, I + 1>(rsrc, lds, voffset);
  }
}

// One 16-key group (16 rows x 64 bytes) of each of N 32-dim blocks.
template <int N, int I = 0>
FA_DEV void dma_blocks(__amdgpu_buffer_rsrc_t rsrc, char* lds, int voffset) {
  if constexpr (I < N) {
    dma16<64 * I>(rsrc, lds + I * PF_VBLOCK_BYTES, voffset);
    dma_blocks<N, I + 1>(rsrc, lds, voffset);
  }
}

FA_DEV u32x4 lds_read16(const char* base, int off) { return *(const u32x4*)(base + off); }
FA_DEV u32x2 lds_read_tr(const char* base, int off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + off)));
}

// The request of rank `rank` when the batch (at most 64 requests) is ordered
// by decreasing key count, ties by index.  Lane i ranks request i; every
// wave computes the same answer.
FA_DEV int64_t request_by_rank(const fa_attn_args& a, int64_t rank, int lane) {
  const int n = (int)a.batch;
  int len = -1;
  if (lane < n) {
    len = a.seqused_k ? a.seqused_k[lane * a.used_k_stride]
                      : a.cu_seqlens_k[(lane + 1) * a.cu_k_stride] - a.cu_seqlens_k[lane * a.cu_k_stride];
  }
  int r = 0;
  for (int j = 0; j < n; ++j) {
    const int lj = __builtin_amdgcn_readlane(len, j);
    r += (lj > len || (lj == len && j < lane)) ? 1 : 0;
  }
  const uint64_t hit = __ballot(lane < n && r == rank);
  return (int64_t)__builtin_ctzll(hit);
}

// V column parts of a tile: 256-dim heads run in 256/128 tiles, each work
// item as two workgroups, one per 128-column half of V and of the output.
template <int DQ, int DV> constexpr int prefill_vparts() { return DQ == 256 && DV == 128 ? 2 : 1; }

struct PrefillShape {
  int n_qblocks;
  int log2_page;   // paged K/V: page of position p = p >> log2_page, slot p & (2^log2_page - 1)
  int compact;     // 1: workgroups map onto the compact work list
  int hp;          // query heads per workgroup (1 or 2, dividing the GQA group): W / hp waves per head
};

// One workgroup's share of the compact work list.  With g = gcd(Hkv, 8),
// XCD x owns the m = Hkv / g KV heads congruent to x mod g of every request,
// and the S = 8 / g XCDs that share those heads take every S-th query block
// of each (counted from the heaviest, phase x / g): Hkv a multiple of 8
// gives heads x, x + 8, ... and S = 1; every XCD sees every request.
// Requests come in order of decreasing key count (ties by index), and
// request b contributes m KV heads x the XCD's query blocks x G workgroups,
// ordered KV head, then query block heaviest-first, then query head.  Slots past the end of the list get no
// item.  Lane l evaluates requests
// l, l + 64, ... (R per lane: at most 64 R requests); the ranking visits
// only requests with query blocks (a mixed batch's single-query requests
// have none).  Every wave computes the same answer.
constexpr int PF_COMPACT_MAX_BATCH = 256;

struct WorkItem {
  int64_t b;
  int qb, kh, g;
  RequestInfo r;
};

// BMH: query rows per head of a workgroup; G: workgroups per query block and
// KV head (the GQA group over the heads packed into one workgroup).
template <int BMH, int R>
FA_DEV bool compact_item(const fa_attn_args& a, int slot, int xcd, int lane, int G, WorkItem& w) {
  const int n = (int)a.batch;
  const int hk = (int)a.heads_k, gk = hk % 8 == 0 ? 8 : hk % 4 == 0 ? 4 : hk % 2 == 0 ? 2 : 1;   // gcd(Hkv, 8)
  const int S = 8 / gk, ph = xcd / gk;   // XCDs sharing a KV head, this XCD's phase
  int qbeg[R], qlen[R], klen[R], kbase[R], nqb[R], nqx[R], before[R];
#pragma unroll
  for (int c = 0; c < R; ++c) {
    const int i = lane + 64 * c;
    qbeg[c] = 0, qlen[c] = 0, klen[c] = -1, kbase[c] = 0, before[c] = 0;
    if (i < n) {
      qbeg[c] = a.cu_seqlens_q[i * a.cu_q_stride];
      qlen[c] = a.cu_seqlens_q[(i + 1) * a.cu_q_stride] - qbeg[c];
      const int kc = a.cu_seqlens_k ? a.cu_seqlens_k[i * a.cu_k_stride] : 0;
      kbase[c] = a.page_size ? 0 : kc;
      klen[c] = a.seqused_k ? a.seqused_k[i * a.used_k_stride] : a.cu_seqlens_k[(i + 1) * a.cu_k_stride] - kc;
    }
    const bool skip = (a.flags & FA_FLAG_SKIP_SINGLE_QUERY) && qlen[c] == 1;   // the decode kernel owns it
    nqb[c] = (i < n && !skip) ? (qlen[c] + BMH - 1) / BMH : 0;
    nqx[c] = nqb[c] > ph ? (nqb[c] - ph + S - 1) / S : 0;   // this XCD's blocks of the request
  }
  // Query blocks of the requests ranked ahead of each of this lane's requests.
#pragma unroll
  for (int cj = 0; cj < R; ++cj) {
    for (uint64_t m = __ballot(nqx[cj] > 0); m; m &= m - 1) {
      const int lj = __builtin_ctzll(m), j = 64 * cj + lj;
      const int kj = __builtin_amdgcn_readlane(klen[cj], lj);
      const int nj = __builtin_amdgcn_readlane(nqx[cj], lj);
#pragma unroll
      for (int c = 0; c < R; ++c)
        before[c] += (kj > klen[c] || (kj == klen[c] && j < lane + 64 * c)) ? nj : 0;
    }
  }
  const int per_block = (hk / gk) * G;
#pragma unroll
  for (int c = 0; c < R; ++c) {
    const int lo = before[c] * per_block;
    const uint64_t hit = __ballot(nqx[c] > 0 && slot >= lo && slot < lo + nqx[c] * per_block);
    if (hit == 0) continue;
    const int l = __builtin_ctzll(hit);
    const int nq = __builtin_amdgcn_readlane(nqb[c], l), nx = __builtin_amdgcn_readlane(nqx[c], l);
    const int t = slot - __builtin_amdgcn_readlane(lo, l);
    const int t2 = t % (nx * G);
    w.b = 64 * c + l;
    w.kh = xcd % gk + gk * (t / (nx * G));
    w.qb = nq - 1 - (ph + S * (t2 / G));
    w.g = t2 % G;
    w.r.q_begin = __builtin_amdgcn_readlane(qbeg[c], l);
    w.r.q_len = __builtin_amdgcn_readlane(qlen[c], l);
    w.r.k_len = __builtin_amdgcn_readlane(klen[c], l);
    w.r.k_base = __builtin_amdgcn_readlane(kbase[c], l);
    w.r.left = a.leftpad_k ? load_invariant_i32(a.leftpad_k, w.b * a.leftpad_stride) : 0;
    w.r.causal = a.causal_by_batch ? a.causal_by_batch[w.b * a.causal_stride] != 0 : a.causal != 0;
    return true;
  }
  return false;
}

// DQ / DV are the tile's head dims (multiples of 64); DQT / DVT <= them are
// the tensors' own (multiples of 8): the query's extra dims load as zero,
// their K columns are never multiplied (K-steps past DQT are skipped, a half
// step is masked), and extra output columns are not stored.
// WIN: sliding windows (a.window_left / a.window_right); without it they are
// ignored and the window code folds away.
// KT: K/V storage type, T or E4M3 (FP8 tiles are staged in LDS and widened
// exactly to T there; k/v descales scale the scores and the output).
// ALIBI: linear biases -slope[b][h] |q_pos - k_pos| seeded into the score
// accumulators (instantiated without softcap, which would come first)
// (flash_attn_mps/kernels/attention.metal:47-51, 87).
// QT: query storage type, T or E4M3.  E4M3 queries (with E4M3 K/V) compute
// S = K Q^T on v_mfma_f32_32x32x64_f8f6f4 with K kept as raw bytes in LDS;
// V is staged and widened exactly to T for O += V P (P stays 16-bit).
// MK: vLLM mask kind (a.mask_kind; 0 none): each row's visible keys are at
// most two key ranges (see mask_ranges below); causality and the window
// fields do not apply, as in the reference (kernels/attention.metal:29-45).
template <typename T, int DQ, int DV, int W, int NB, int MINB, bool CAUSAL, bool CAP, bool WIN, int DQT = DQ,
          int DVT = DV, typename KT = T, bool ALIBI = false, typename QT = T, int MK = 0>
__global__ __launch_bounds__(64 * W, MINB) void prefill_kernel(const fa_attn_args a, const PrefillShape shp) {
  static_assert(MK == 0 || (!CAUSAL && !WIN && !ALIBI), "mask kinds carry their own causality and windows");
  constexpr bool GEN = WIN || MK != 0;   // per-stage hot / masked decisions (no closed-form hot loop)
  constexpr bool FP8 = KT::id == FA_E4M3;
  constexpr bool FQ = QT::id == FA_E4M3;       // E4M3 queries: FP8 MFMA for S
  // ALiBi without softcap is folded into the score accumulators before the
  // MFMAs (raw dot-product units); with softcap it follows the softcap.
  constexpr bool ALIBI_FOLD = ALIBI && !CAP, ALIBI_LATE = ALIBI && CAP;
  constexpr int KEB = KT::bytes;               // bytes per K/V element
  static_assert(!FP8 || (DQT == DQ && DVT == DV && ((DQ == DV && (DQ == 64 || DQ == 128 || DQ == 256)) ||
                                                      (DQ == 256 && DV == 128))),
                "FP8 K/V tiles: 64/128/256-dim heads (256-dim: also as 256/128 V halves)");
  static_assert(!FQ || FP8, "E4M3 queries: E4M3 K/V");
  constexpr int BM = 32 * NB * W;              // query rows per workgroup
  constexpr int KST = DQ / 16;                 // k-steps of the QK^T MFMA
  constexpr int KSTT = (DQT + 15) / 16;        // k-steps holding real dims
  static_assert(DQT % 8 == 0 && DVT % 8 == 0 && DQT <= DQ && DVT <= DV, "true head dims");
  constexpr int DB = DV / 32;                  // 32-dim blocks of O^T
  constexpr int KG = DQ / 64, VG = DV / 64;    // 64-dim column groups (K), pairs of 32-dim blocks (V)
  // A K tile is KGD 128-byte-row column groups: 64 bf16 dims each, or 128
  // E4M3 dims (E4M3 queries keep K raw; a 64-dim head fills half of its
  // group's rows, the other half holds whatever follows the row in memory,
  // or zeros past the request, and is never read).
  constexpr int KGD = FQ ? (DQ + 127) / 128 : KG;
  constexpr int KTILE = KGD * PF_GROUP_BYTES, VTILE = VG * PF_GROUP_BYTES;
  static_assert(DQ % 64 == 0 && DV % 64 == 0, "head dims are multiples of 64");
  static_assert(W == 2 || W == 4 || W == 8, "wave count");

  extern __shared__ __attribute__((aligned(16))) char smem[];
  char* const kbuf0 = smem;
  char* const vbuf0 = smem + 2 * KTILE;
  // FP8: one staging tile of raw K and V rows (64 x DQ and 64 x DV bytes);
  // E4M3 queries: two staging tiles of raw V rows only.
  char* const stk = smem + 2 * KTILE + 2 * VTILE;
  char* const stv = FQ ? stk : stk + 64 * DQ;

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave_u = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index as a scalar
  // Work order.  Workgroups are dispatched round-robin over the 8 XCDs
  // (XCD = blockIdx % 8), each with its own L2, and every XCD works through
  // whole (request, KV head) pairs one after another, query blocks
  // heaviest-first, so the resident workgroups of an XCD share K/V in its L2.
  // Requests come longest first (batches of up to 64), so the grid ends on
  // the blocks of short requests rather than on the heavy blocks of a long
  // one.  Compact mode launches only real work; otherwise XCD x takes the
  // pairs p = x, x + 8, ... with n_qblocks slots each and skips the slots
  // past a request's end.
  // With hp = 2 a workgroup holds BM / 2 rows of two query heads of one KV
  // head (waves 0 .. W/2-1 the first head), sharing every K/V tile.
  // V column parts (prefill_vparts = 2): the head's V and output columns are two
  // halves of DVT, each a workgroup of its own that recomputes S (a 256-dim
  // head then holds half of O^T, within the 256 registers of two waves per
  // SIMD).  Blocks 16j..16j+7 take half 0 and 16j+8..16j+15 half 1 of work
  // slots 8j..8j+7: both halves of an item run on one XCD, next to each
  // other in dispatch order (their Q and K reads still mostly come from HBM
  // twice: 1.68x the algorithmic bytes on config 2's lengths at d256).
  constexpr bool TWO_PARTS = prefill_vparts<DQ, DV>() == 2;
  const int vpart = TWO_PARTS ? (int)(blockIdx.x >> 3) & 1 : 0;
  const unsigned bid = TWO_PARTS ? (blockIdx.x >> 4) << 3 | (blockIdx.x & 7) : blockIdx.x;
  const int G = (int)(a.heads_q / a.heads_k) / shp.hp;
  const int xcd = bid % 8, slot = bid / 8;
  WorkItem wi;
  if (shp.compact) {
    bool found;
    if (a.batch <= 64)
      found = shp.hp == 2 ? compact_item<BM / 2, 1>(a, slot, xcd, lane, G, wi) : compact_item<BM, 1>(a, slot, xcd, lane, G, wi);
    else
      found = shp.hp == 2 ? compact_item<BM / 2, PF_COMPACT_MAX_BATCH / 64>(a, slot, xcd, lane, G, wi)
                          : compact_item<BM, PF_COMPACT_MAX_BATCH / 64>(a, slot, xcd, lane, G, wi);
    if (!found) return;
  } else {
    const int per_pair = shp.n_qblocks * G;
    const int64_t pair = (int64_t)(slot / per_pair) * 8 + xcd;
    if (pair >= a.batch * a.heads_k) return;
    const int rem = slot % per_pair;
    wi.qb = shp.n_qblocks - 1 - rem / G;
    wi.g = rem % G;
    wi.b = a.batch > 1 && a.batch <= 64 ? request_by_rank(a, pair / a.heads_k, lane) : pair / a.heads_k;
    wi.kh = (int)(pair % a.heads_k);
    wi.r = load_request(a, wi.b);
    if ((a.flags & FA_FLAG_SKIP_SINGLE_QUERY) && wi.r.q_len == 1) return;   // the decode kernel owns it
  }
  const int64_t b = wi.b;
  const int wph = W / shp.hp;   // waves per head
  const int bmh = 32 * NB * wph;   // query rows per head
  const int qb = wi.qb, kh = wi.kh, h = (kh * G + wi.g) * shp.hp + wave_u / wph;
  const RequestInfo r = wi.r;
  const int q0 = qb * bmh;
  if (q0 >= r.q_len) return;
  const int off = r.k_len - r.q_len;   // absolute position of query row i is i + off
  const int wq0 = q0 + (wave_u % wph) * 32 * NB;   // this wave's first query row
  auto wq0_of = [&](int nb) { return wq0 + 32 * nb + l32; };   // this lane's row of block nb
  // Row qa sees keys j with qa - WL <= j (WL >= 0), j <= qa (causal) or
  // j <= qa + WR (WR >= 0, not causal), j < k_len (flash_attn_mps/kernels/
  // attention.metal:29-45, window kind).  The workgroup's key range follows
  // from its first and last rows.
  // Per-request causality (a.causal_by_batch) runs in the non-causal WIN
  // variant: a causal request is the right window 0.
  const int WL = WIN ? a.window_left : -1, WR = (WIN && !CAUSAL) ? (r.causal ? 0 : a.window_right) : -1;
  const int qa_first = q0 + off, qa_last = min(q0 + bmh, r.q_len) - 1 + off;
  int kv_end = r.k_len;
  if (CAUSAL) kv_end = min(kv_end, qa_last + 1);
  else if (WR >= 0) kv_end = min(kv_end, max(qa_last + WR + 1, 0));
  int kv_begin = WL >= 0 ? min(max(qa_first - WL, 0), max(kv_end, 0)) : 0;

  // Mask kinds (flash_attn_mps/kernels/attention.metal:29-45), with qa the
  // row's absolute position and keys below k_len:
  //   kind 1 (vllm.mm_prefix_mask): [qa - W + 1, qa] (W = a.mask_window,
  //     [0, qa] when W < 0) and the row's modality range [lo, hi] =
  //     a.mask_ranges[row] when lo >= 0 (from qa - W + 1 on with
  //     a.mask_clamp);
  //   kind 2 (vllm.rswa_mask): [0, min(P - 1, qa)] with P = a.mask_prefix[b]
  //     and [qa - Wl + 1, qa] with Wl = a.mask_window_len[0].
  // mr[nb] = {a1, b1, a2, b2}: the two ranges of this lane's row of block nb
  // (absolute keys, a > b when empty).  Kind 2 runs the key pipeline once per
  // range when the two are apart for every row of the workgroup (the keys
  // between them are never loaded), each run with one range.
  constexpr int PF_FAR = 1 << 29;   // beyond any key (the host bounds k_len)
  int mr[NB][4];
  int mk_p = 0, mk_w = 0;           // kind 2: prefix length, window
  bool mk_split = false;            // kind 2: two runs
  auto clip_hi = [&](int x) { return min(x, r.k_len - 1); };
  auto set_ranges = [&](int part) {  // kind 2: 0 both ranges, 1 the prefix only, 2 the window only
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int row = wq0_of(nb), qa = row + off;
      int a1 = PF_FAR, b1 = -PF_FAR, a2 = PF_FAR, b2 = -PF_FAR;
      if (row < r.q_len) {
        if constexpr (MK == 1) {
          const int wm = a.mask_window;
          a1 = wm > 0 ? max(qa - wm + 1, 0) : 0;
          b1 = clip_hi(qa);
          const int64_t tq = (int64_t)r.q_begin + row;
          const int lo = a.mask_ranges[tq * a.ranges_stride[0]];
          const int hi = a.mask_ranges[tq * a.ranges_stride[0] + a.ranges_stride[1]];
          if (lo >= 0) {
            a2 = (a.mask_clamp && wm > 0) ? max(lo, qa - wm + 1) : lo;
            b2 = clip_hi(hi);
          }
        } else if constexpr (MK == 2) {
          if (part != 2) {
            a1 = 0;
            b1 = clip_hi(min(mk_p - 1, qa));
          }
          if (part != 1) {
            a2 = max(max(qa - mk_w + 1, 0), part == 2 ? mk_p : 0);
            b2 = clip_hi(qa);
          }
        }
      }
      mr[nb][0] = a1, mr[nb][1] = b1, mr[nb][2] = a2, mr[nb][3] = b2;
    }
  };
  if constexpr (MK == 1) {
    // Key range of the workgroup: its rows' windows and modality ranges.
    int lo_min = PF_FAR, hi_max = -1;
    for (int i = lane; i < bmh; i += 64) {
      const int row = q0 + i;
      if (row < r.q_len) {
        const int64_t tq = (int64_t)r.q_begin + row;
        const int lo = a.mask_ranges[tq * a.ranges_stride[0]];
        const int hi = a.mask_ranges[tq * a.ranges_stride[0] + a.ranges_stride[1]];
        if (lo >= 0 && hi >= lo) {
          lo_min = min(lo_min, lo);
          hi_max = max(hi_max, hi);
        }
      }
    }
    lo_min = __builtin_amdgcn_readfirstlane(wave_min_i(lo_min));
    hi_max = __builtin_amdgcn_readfirstlane(wave_max_i(hi_max));
    kv_end = min(r.k_len, max(qa_last + 1, hi_max + 1));
    kv_begin = a.mask_window > 0 ? max(min(qa_first - a.mask_window + 1, lo_min), 0) : 0;
    kv_begin = min(kv_begin, max(kv_end, 0));
  } else if constexpr (MK == 2) {
    mk_p = load_invariant_i32(a.mask_prefix, b * a.prefix_stride);
    mk_w = load_invariant_i32(a.mask_window_len, 0);
    kv_end = min(r.k_len, qa_last + 1);
    const int wfirst = max(qa_first - mk_w + 1, 0);   // first key of the earliest row's window
    // Apart when no key between the prefix and the windows is visible:
    // whole 64-key tiles lie between them.
    mk_split = mk_p > 0 && (mk_p + PF_BN - 1) / PF_BN < wfirst / PF_BN;
    kv_begin = mk_p > 0 ? 0 : min(wfirst, max(kv_end, 0));
  }
  int n_tiles = kv_end > 0 ? (kv_end + PF_BN - 1) / PF_BN : 0;
  int tile0 = kv_begin / PF_BN;   // first tile with a visible key

  // Descales (per request and KV head, 1 when absent): score = scale *
  // q_descale * k_descale * q.k, output * v_descale
  // (flash_attn_mps/kernels/attention.metal:47-51, 170-180).  A negative
  // score scale is carried by Q's sign bits (flipped once below), so the
  // kernel's scale is positive and the row max of the raw dot products is
  // the row max of the scores.
  const float kdsc = descale_of(a.q_descale, a.q_descale_stride, b, kh) *
                     descale_of(a.k_descale, a.k_descale_stride, b, kh);
  const float vdsc = descale_of(a.v_descale, a.v_descale_stride, b, kh);
  const bool q_flip = a.softmax_scale * kdsc < 0.0f;
  float kscale = q_flip ? -(a.softmax_scale * kdsc) : a.softmax_scale * kdsc;
  const uint32_t q_flip16 = q_flip ? 0x80008000u : 0u, q_flip8 = q_flip ? 0x80808080u : 0u;   // sign bits
  // The folded ALiBi bias is in raw units (slope / scale): with a zero score
  // scale every dot product is replaced by 0 (Q zeroed) and the fold uses a
  // unit scale, so the scores are the biases alone, as in the reference.
  const bool q_zero = ALIBI_FOLD && !(kscale > 0.0f);
  if (q_zero) kscale = 1.0f;
  const uint32_t q_keep = q_zero ? 0u : 0xffffffffu;

  // Q^T operands for the whole kernel: block nb, lane holds
  // Q[wq0 + 32 nb + l32][16 kk + 8 hh .. +8].
  constexpr int KST8 = DQ / 64;                // k-steps of the E4M3 S MFMA
  u32x4 qop[FQ ? 1 : NB][FQ ? 1 : KST];
  i32x8 qop8[FQ ? NB : 1][FQ ? KST8 : 1];      // E4M3: Q[row][64 j + 32 hh .. +32]
  // Rows past the request load its last row (their results are never
  // stored), so every load is unconditional and nothing touches the loaded
  // registers before the first tile's wait: the Q loads' latency overlaps
  // the first K/V DMAs.  (Exec-masked loads with zero defaults made the
  // compiler wait for the first of them before issuing the rest.)  The sign
  // flip and the ALiBi zeroing are rare; a uniform branch applies them.
  const bool q_fix = q_flip || q_zero;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int row = min(wq0 + 32 * nb + l32, r.q_len - 1);
    if constexpr (FQ) {
      const uint8_t* qp = (const uint8_t*)a.q + ((int64_t)r.q_begin + row) * a.q_stride[0] +
                          (int64_t)h * a.q_stride[1] + 32 * hh;
#pragma unroll
      for (int j = 0; j < KST8; ++j) {
        const u32x4 lo = *(const u32x4*)(qp + 64 * j), hi = *(const u32x4*)(qp + 64 * j + 16);
        qop8[nb][j] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
      if (q_fix) {
#pragma unroll
        for (int j = 0; j < KST8; ++j)
#pragma unroll
          for (int e = 0; e < 8; ++e) qop8[nb][j][e] = (int)(((uint32_t)qop8[nb][j][e] ^ q_flip8) & q_keep);
      }
    } else {
      const uint16_t* qp = (const uint16_t*)a.q + ((int64_t)r.q_begin + row) * a.q_stride[0] +
                           (int64_t)h * a.q_stride[1] + 8 * hh;
#pragma unroll
      for (int kk = 0; kk < KST; ++kk) {
        if constexpr (DQT == DQ) {
          qop[nb][kk] = *(const u32x4*)(qp + 16 * kk);
        } else {
          u32x4 v = {0u, 0u, 0u, 0u};
          if (16 * kk + 8 * hh + 8 <= DQT) v = *(const u32x4*)(qp + 16 * kk);
          qop[nb][kk] = v;
        }
      }
      if (q_fix) {
#pragma unroll
        for (int kk = 0; kk < KST; ++kk)
#pragma unroll
          for (int e = 0; e < 4; ++e) qop[nb][kk][e] = (qop[nb][kk][e] ^ q_flip16) & q_keep;
      }
    }
  }

  // Rows past the request's last key are never written by the DMA loads of
  // some hardware paths; zeroed V buffers keep p * v finite for them.
  // (FP8: the staging tile, whose rows are converted whole.)
  if constexpr (FP8) {
    constexpr int STAGE_BYTES = FQ ? 2 * 64 * DV : 64 * (DQ + DV);
    for (int i = tid; i < STAGE_BYTES / 16; i += 64 * W) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      *(u32x4*)(stk + 16 * i) = z;
    }
    __syncthreads();
  } else {
    // Only a buffer whose first tile ends past the request's last key needs
    // it (later tiles find the finite rows of earlier ones); without mask
    // kinds the first tiles are tile0 and tile0 + 1.
    const bool need = MK != 0 || (tile0 + 1) * PF_BN > r.k_len || (tile0 + 1 < n_tiles && (tile0 + 2) * PF_BN > r.k_len);
    if (need) {
      for (int i = tid; i < 2 * VTILE / 16; i += 64 * W) {
        const u32x4 z = {0u, 0u, 0u, 0u};
        *(u32x4*)(vbuf0 + 16 * i) = z;
      }
      __syncthreads();
    }
  }

  // ---- DMA addressing.  A tile is 8 row blocks (8 rows each) per column
  // group; one instruction moves one row block of one column group.  Lane p
  // fills LDS row 8 rb + p / 8, 16-byte slot p % 8, which holds chunk
  // (p % 8) ^ ((row / 2) % 8) of that row; K rows hold key sigma(row).
  // Offsets are relative to the first key of the row's 16-key group, whose
  // address the per-group descriptor carries.  Wave w owns K row blocks
  // rb = w + W i: all have rb % 2 = w % 2, so one lane offset serves them all
  // and the column group is an immediate.  V: one instruction moves one
  // 16-key group of one 32-dim block (16 rows x 64 bytes, lane p -> row
  // p / 4, chunk p % 4); wave w owns the groups w + W i, the block is an
  // immediate.
  const bool paged = a.page_size != 0;
  const int lp = shp.log2_page;
  const int drow = 8 * (wave_u & 1) + (lane >> 3);   // row within its 16-key group
  const int kdoff = KEB * (int)(sigma(drow) * a.k_stride[1]) + (((lane & 7) ^ ((drow >> 1) & 7)) * 16);
  const int vdoff = 2 * (int)((lane >> 2) * a.v_stride[1]) + (lane & 3) * 16;
  const char* const khead = (const char*)a.k + KEB * (int64_t)kh * a.k_stride[2];
  // (readfirstlane: the part's column offset stays a scalar, as the
  // descriptors built from vhead must)
  const char* vhead = (const char*)a.v + KEB * (int64_t)kh * a.v_stride[2];
  if constexpr (TWO_PARTS) vhead += __builtin_amdgcn_readfirstlane(vpart * DVT * KEB);
  const uint32_t krow_b = (uint32_t)(KEB * a.k_stride[1]), vrow_b = (uint32_t)(KEB * a.v_stride[1]);
  const uint32_t kpage_b = (uint32_t)(KEB * a.k_stride[0]), vpage_b = (uint32_t)(KEB * a.v_stride[0]);
  const int32_t* const trow = paged ? a.block_table + b * a.bt_stride[0] : nullptr;
  const int bt1 = (int)a.bt_stride[1];
  const int pmask = (1 << lp) - 1;
  // Descriptor of the 16-key group starting at key0: base = that key's row,
  // size ends at the request's last key (0 bytes for groups past it).
  auto group_rsrc = [&](const char* head, uint32_t row_b, uint32_t page_b, int key0, int row_bytes) {
    const int nvalid = min(max(r.k_len - key0, 0), 16);
    const char* g = head;
    if (nvalid > 0) {
      const int pos = key0 + r.left;   // storage position (leftpad: a dense cache's hidden prefix)
      if (paged) {
        const uint32_t blk = (uint32_t)load_invariant_i32(trow, (int64_t)(pos >> lp) * bt1);
        g = head + (uint64_t)blk * page_b + (uint32_t)(pos & pmask) * row_b;
      } else {
        g = head + (uint64_t)(uint32_t)(r.k_base + pos) * row_b;
      }
    }
    // readfirstlane keeps the (uniform) size in an SGPR: a VGPR-held
    // descriptor field would make the compiler wrap each load in a loop over
    // distinct descriptors.
    const int bytes = __builtin_amdgcn_readfirstlane(nvalid > 0 ? (nvalid - 1) * (int)row_b + row_bytes : 0);
    return __builtin_amdgcn_make_buffer_rsrc((void*)g, (short)0, bytes, 0x00020000);
  };
  // The same for a group known to hold 16 keys of the request: scalar
  // arithmetic only, size = 16 rows; pg (paged or not) is a compile-time tag.
  const int knrec = 15 * (int)krow_b + KEB * DQT, vnrec = 15 * (int)vrow_b + KEB * DVT;
  auto full_rsrc = [&](auto pg, const char* head, uint32_t row_b, uint32_t page_b, int key0, int nrec) {
    const char* g;
    const int pos = key0 + r.left;
    if constexpr (decltype(pg)::value) {
      const uint32_t blk = (uint32_t)load_invariant_i32(trow, (int64_t)(pos >> lp) * bt1);
      g = head + (uint64_t)blk * page_b + (uint32_t)(pos & pmask) * row_b;
    } else {
      g = head + (uint64_t)(uint32_t)(r.k_base + pos) * row_b;
    }
    return __builtin_amdgcn_make_buffer_rsrc((void*)g, (short)0, nrec, 0x00020000);
  };
  auto paged_tag = [](auto mode) { return std::integral_constant<bool, decltype(mode)::value == PF_FULL_PAGED>(); };
  // Load modes (a compile-time tag): PF_ANY_TILE = any tile, per-group
  // bounds; PF_FULL_PACKED / PF_FULL_PAGED = tiles known to hold 64 keys of
  // the request, packed or paged K/V.
  // K rows 32 half .. +32 of a tile (row blocks 4 half .. +4).
  auto dma_k = [&](auto mode, int tile, int buf, int half) {
#pragma unroll
    for (int i = 0; i < 8 / W; ++i) {
      const int rb = wave_u + W * i;
      if ((rb >> 2) != half) continue;
      const int key0 = tile * PF_BN + 16 * (rb >> 1);
      const auto rsrc = decltype(mode)::value == PF_ANY_TILE
                            ? group_rsrc(khead, krow_b, kpage_b, key0, KEB * DQT)
                            : full_rsrc(paged_tag(mode), khead, krow_b, kpage_b, key0, knrec);
      dma_columns<KGD>(rsrc, kbuf0 + buf * KTILE + rb * 1024, kdoff);
    }
  };
  auto dma_v = [&](auto mode, int tile, int buf) {
#pragma unroll
    for (int i = 0; i < (4 + W - 1) / W; ++i) {
      const int gi = wave_u + W * i;
      if (gi >= 4) continue;
      const int key0 = tile * PF_BN + 16 * gi;
      const auto rsrc = decltype(mode)::value == PF_ANY_TILE
                            ? group_rsrc(vhead, vrow_b, vpage_b, key0, KEB * DVT)
                            : full_rsrc(paged_tag(mode), vhead, vrow_b, vpage_b, key0, vnrec);
      dma_blocks<2 * VG>(rsrc, vbuf0 + buf * VTILE + gi * 1024, vdoff);
    }
  };
  // FP8: whole tiles into the staging buffer, 1 KiB (1024 / D rows) per
  // instruction; a wave's instructions n = w + W i each stay inside one
  // 16-key group, at the same row offset within it.
  // The staging rows are stored with their 16-byte chunks permuted (chunk u
  // of row r at position u ^ stage_rows(r), a per-row XOR that stays inside
  // the row): the widening passes below then read them without bank
  // conflicts.
  constexpr int KR8 = 1024 / DQ, VR8 = 1024 / DV;   // rows per instruction
  const int k8row = ((KR8 * wave_u) & 15) + lane / (DQ / 16), v8row = ((VR8 * wave_u) & 15) + lane / (DV / 16);
  const int k8off = k8row * (int)krow_b + ((lane % (DQ / 16)) ^ stage_rows<DQ>(k8row)) * 16;
  const int v8off = v8row * (int)vrow_b + ((lane % (DV / 16)) ^ stage_rows<DV>(v8row)) * 16;
  auto dma_fp8 = [&](int tile) {
#pragma unroll
    for (int i = 0; i < 64 / KR8 / W; ++i) {
      const int n = wave_u + W * i;
      const auto rsrc = group_rsrc(khead, krow_b, kpage_b, tile * PF_BN + ((n * KR8) & ~15), DQ);
      dma16<0>(rsrc, stk + n * 1024, k8off);
    }
#pragma unroll
    for (int i = 0; i < 64 / VR8 / W; ++i) {
      const int n = wave_u + W * i;
      const auto rsrc = group_rsrc(vhead, vrow_b, vpage_b, tile * PF_BN + ((n * VR8) & ~15), DV);
      dma16<0>(rsrc, stv + n * 1024, v8off);
    }
  };
  // E4M3 queries: V tile -> staging slot `slot` (two 64 x DV byte tiles).
  auto dma_v8 = [&](int tile, int slot) {
#pragma unroll
    for (int i = 0; i < 64 / VR8 / W; ++i) {
      const int n = wave_u + W * i;
      const auto rsrc = group_rsrc(vhead, vrow_b, vpage_b, tile * PF_BN + ((n * VR8) & ~15), DV);
      dma16<0>(rsrc, stv + slot * 64 * DV + n * 1024, v8off);
    }
  };
  // Staging -> tile buffers, widened exactly to T.  Each 16-lane group
  // converts 16-byte staging chunks (16 E4M3 values -> 32 bytes of T) of 4
  // consecutive keys x 4 consecutive chunks: one 64-dim K column group, or
  // two 32-dim V blocks.  Every lane writes its two 16-byte halves in an
  // order that depends on the lane, so each 8-lane write cycle covers 8
  // distinct slots: K rows r and r + 1 share a swizzle, so odd keys write
  // their upper half first; V rows are 64 bytes, so the second block of the
  // pair writes its upper half first.  (A mapping by consecutive staging
  // chunks conflicted 2-4 ways on K and 4-8 ways on V writes.)  The lane
  // swaps the two 8-byte halves of its staging chunk before converting (4
  // selects), rather than the two converted halves after it (8).  The
  // addresses derive from an opaque copy of t so that none of them is held
  // in registers across the main loop.
  static_assert(!FP8 || (DQ % (16 * W) == 0 && DV % (16 * W) == 0), "FP8 widening: whole groups per pass");
  auto widen_k_rows = [&](int t, int buf) {
    constexpr int NG = DQ / 64, GPI = 64 * W / 16;   // column groups; 16-lane groups per pass
    const int l16 = t & 15, m = l16 & 3, g = (t >> 4) % NG;
#pragma unroll
    for (int it = 0; it < DQ / (16 * W); ++it) {
      const int q = (it * GPI + (t >> 4)) / NG;
      const int r = 4 * q + (l16 >> 2), u = 4 * g + m, rho = sigma(r), sw = (rho >> 1) & 7, up = r & 1;
      u32x4 first, second;
      widen_fp8_16<T>(halves_swapped_if(*(const u32x4*)(stk + r * DQ + 16 * (u ^ stage_rows<DQ>(r))), up), first,
                      second);
      char* const row = kbuf0 + buf * KTILE + g * PF_GROUP_BYTES + rho * 128;
      *(u32x4*)(row + ((2 * m + up) ^ sw) * 16) = first;
      *(u32x4*)(row + ((2 * m + 1 - up) ^ sw) * 16) = second;
    }
  };
  auto widen_v_rows = [&](int t, const char* stage, int buf) {
    constexpr int NC = DV / 64, GPI = 64 * W / 16;   // 64-dim block pairs; 16-lane groups per pass
    const int l16 = t & 15, c = (t >> 4) % NC, up = (l16 >> 1) & 1, h = l16 & 1;
    const int blk = 2 * c + up, u = 4 * c + (l16 & 3);
#pragma unroll
    for (int it = 0; it < DV / (16 * W); ++it) {
      const int r = 4 * ((it * GPI + (t >> 4)) / NC) + (l16 >> 2);
      u32x4 first, second;
      widen_fp8_16<T>(halves_swapped_if(*(const u32x4*)(stage + r * DV + 16 * (u ^ stage_rows<DV>(r))), up), first,
                      second);
      char* const dst = vbuf0 + buf * VTILE + blk * PF_VBLOCK_BYTES + r * 64 + 32 * h;
      *(u32x4*)(dst + 16 * up) = first;
      *(u32x4*)(dst + 16 * (1 - up)) = second;
    }
  };
  // E4M3 queries: staging slot -> V buffer buf.
  auto widen_v = [&](int slot, int buf) {
    int t = tid;
    asm volatile("" : "+v"(t));
    widen_v_rows(t, stv + slot * 64 * DV, buf);
  };
  // FP8 K/V: staging -> tile buffer buf in the 16-bit layouts above (K: key r
  // at row sigma(r), swizzled 8-dim chunks; V: 32-dim blocks).
  auto widen_tile = [&](int buf) {
    int t = tid;
    asm volatile("" : "+v"(t));
    widen_k_rows(t, buf);
    widen_v_rows(t, stv, buf);
  };

  // ---- Operand read offsets (bytes within a tile buffer).
  // K (A of S^T): LDS row 32 (st % 2) + l32, chunk 2 kk + hh -> column group
  // kk / 4, slot (2 (kk % 4) + hh) ^ ((l32 / 2) % 8); kk / 4 is an immediate.
  int krd[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) krd[s] = l32 * 128 + (((2 * s + hh) ^ ((l32 >> 1) & 7)) * 16);
  // E4M3 K (A of S^T, 64 dims per step): step j reads chunks 4 (j % 2) + 2 hh
  // and + 1 of column group j / 2; index 2 (j % 2) + e.
  int krd8[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) krd8[s] = l32 * 128 + (((4 * (s >> 1) + 2 * hh + (s & 1)) ^ ((l32 >> 1) & 7)) * 16);
  // V^T (A of O^T) through ds_read_b64_tr_b16: in each 16-lane group g, lane
  // i = a + 4 t' reads row 8 (g / 2) + t' (+ 32 (st % 2) + 16 c + 4 t) of
  // block db at dims 16 (g % 2) + 4 a .. +4; the hardware hands lane 4 a + e
  // dim 4 a + e of those four rows, i.e. four consecutive keys of one dim.
  const int vg16 = lane >> 4, vi = lane & 15, va = vi & 3, vt = vi >> 2;
  const int vrd = (8 * (vg16 >> 1) + vt) * 64 + (4 * (vg16 & 1) + va) * 8;

  const float c_scale = kscale * LOG2E;   // raw dot -> log2 units
  const float cap_in = CAP ? 2.0f * LOG2E * kscale / a.softcap : 0.0f;
  const float cap_out = a.softcap * LOG2E;
  // ALiBi slope: folded, in raw dot-product units (the score's bias
  // -slope |qa - key| becomes -sl |qa - key| before the scale, kscale > 0);
  // after the softcap, in log2 units.
  const float slope = ALIBI ? a.alibi[b * a.alibi_stride[0] + (int64_t)h * a.alibi_stride[1]] : 0.0f;
  const float sl = ALIBI_FOLD ? slope / kscale : 0.0f;
  const float sl2 = ALIBI_LATE ? slope * LOG2E : 0.0f;
  // A sink logit seeds the running state (max = sink, sum = 1) of every row.
  const float sink2 = a.sinks ? a.sinks[(int64_t)h * a.sink_stride] * LOG2E : -INFINITY;
  float m_run[NB], l_run[NB];
  f32x16 o[NB][DB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    m_run[nb] = sink2;
    l_run[nb] = (a.sinks && hh == 0) ? 1.0f : 0.0f;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[nb][db][i] = 0.0f;
  }

  const bool wave_rows = wq0 < r.q_len;
  const int wave_qabs_lo = wq0 + off;
  const int wave_qabs_hi = min(wq0 + 32 * NB, r.q_len) - 1 + off;
  // The pipeline runs over 32-key stages: stage st is half st % 2 of tile
  // st / 2 (keys 32 st .. +32).
  int n_stages = kv_end > 0 ? (kv_end + 31) / 32 : 0;
  int st0 = 2 * tile0;
  // Keys some row of this wave sees: [wave_key_lo, wave_key_hi].
  const int wave_key_lo = WL >= 0 ? wave_qabs_lo - WL : INT_MIN;
  const int wave_key_hi = CAUSAL ? wave_qabs_hi : (WR >= 0 ? wave_qabs_hi + WR : INT_MAX);
  // Mask kinds: keys some row of this wave sees, [wu_lo, wu_hi], and the
  // keys of range 1 / range 2 every row of it sees, [wf1a, wf1b] / [wf2a,
  // wf2b] (from mr; rows past the request constrain nothing).
  int wu_lo = PF_FAR, wu_hi = -PF_FAR, wf1a = 0, wf1b = -1, wf2a = 0, wf2b = -1;
  auto wave_bounds = [&]() {
    int ulo = PF_FAR, uhi = -PF_FAR, f1a = -PF_FAR, f1b = PF_FAR, f2a = -PF_FAR, f2b = PF_FAR;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (wq0_of(nb) < r.q_len) {
        if (mr[nb][0] <= mr[nb][1]) ulo = min(ulo, mr[nb][0]), uhi = max(uhi, mr[nb][1]);
        if (mr[nb][2] <= mr[nb][3]) ulo = min(ulo, mr[nb][2]), uhi = max(uhi, mr[nb][3]);
        f1a = max(f1a, mr[nb][0]), f1b = min(f1b, mr[nb][1]);
        f2a = max(f2a, mr[nb][2]), f2b = min(f2b, mr[nb][3]);
      }
    }
    // Wave-uniform after the reductions; readfirstlane keeps them in SGPRs.
    wu_lo = __builtin_amdgcn_readfirstlane(wave_min_i(ulo));
    wu_hi = __builtin_amdgcn_readfirstlane(wave_max_i(uhi));
    wf1a = __builtin_amdgcn_readfirstlane(wave_max_i(f1a));
    wf1b = __builtin_amdgcn_readfirstlane(wave_min_i(f1b));
    wf2a = __builtin_amdgcn_readfirstlane(wave_max_i(f2a));
    wf2b = __builtin_amdgcn_readfirstlane(wave_min_i(f2b));
  };
  auto active = [&](int st) {
    if constexpr (MK != 0) return wave_rows && st * 32 + 31 >= wu_lo && st * 32 <= wu_hi;
    else return wave_rows && st * 32 <= wave_key_hi && st * 32 + 31 >= wave_key_lo;
  };
  auto needs_mask = [&](int st) {
    const int t0 = st * 32;
    if constexpr (MK != 0) return !((t0 >= wf1a && t0 + 31 <= wf1b) || (t0 >= wf2a && t0 + 31 <= wf2b));
    else
      return (t0 + 32 > r.k_len) || (CAUSAL && t0 + 31 > wave_qabs_lo) || (WL >= 0 && t0 < wave_qabs_hi - WL) ||
             (WR >= 0 && t0 + 31 > wave_qabs_lo + WR);
  };

  // S^T of one stage: s[nb][i] = score of key 32 st + 16 (i >> 3) + 8 hh + (i & 7).
  // With ALiBi the accumulators start at the key's bias, so the MFMAs add
  // the dot product onto it: -sl |x| with x = key - qa, which is sl x on
  // every key a causal row sees (keys past the row are masked later).
  // par: std::integral_constant<int, 2 p + e> when stage st is known to be
  // half e of a tile in K/V buffer p (the LDS reads then take the stage's
  // rows as immediate offsets), or <int, -1> (from st at run time).
  auto qk = [&](int st, f32x16 (&s)[NB], auto par) {
    constexpr int PAR = decltype(par)::value;
    const char* kl;
    if constexpr (PAR < 0) kl = kbuf0 + ((st >> 1) & 1) * KTILE + (st & 1) * 32 * 128;
    else kl = kbuf0 + (PAR >> 1) * KTILE + (PAR & 1) * 32 * 128;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if constexpr (ALIBI_FOLD) {
        const float d = (float)(st * 32 + 8 * hh - (wq0 + 32 * nb + l32 + off));
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float x = d + (float)(16 * (i >> 3) + (i & 7));
          s[nb][i] = CAUSAL ? sl * x : -sl * fabsf(x);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) s[nb][i] = 0.0f;
      }
    }
    if constexpr (FQ) {
#pragma unroll
      for (int j = 0; j < KST8; ++j) {
        const char* g = kl + (j >> 1) * PF_GROUP_BYTES;
        const u32x4 lo = lds_read16(g, krd8[2 * (j & 1)]), hi = lds_read16(g, krd8[2 * (j & 1) + 1]);
        const i32x8 av = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) s[nb] = mfma32_fp8(av, qop8[nb][j], s[nb]);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < KSTT; ++kk) {
        u32x4 av = lds_read16(kl, krd[kk % 4] + (kk / 4) * PF_GROUP_BYTES);
        if constexpr (DQT % 16 == 8) {
          if (kk == KSTT - 1 && hh) av = u32x4{0u, 0u, 0u, 0u};   // dims past DQT: whatever the DMA read
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) s[nb] = mfma32<T>(av, qop[nb][kk], s[nb]);
      }
    }
  };
  // Phase A: softcap, mask, row max and the lazy rescale of (m, l); fills
  // O's factors, applied before the stage's P.V.  With commit false (a stage
  // past this wave's causal range) the running state is left untouched.
  auto phase_a = [&](auto mask_tag, int st, f32x16 (&s)[NB], bool commit, float (&f)[NB]) {
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if constexpr (CAP) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float e = fast_exp2(cap_in * s[nb][i]);
          s[nb][i] = cap_out * (1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f));
        }
      }
      if constexpr (ALIBI_LATE) {
        // softcap(score) - slope |qa - key|, in log2 units.
        const float d = (float)(st * 32 + 8 * hh - (wq0 + 32 * nb + l32 + off));
#pragma unroll
        for (int i = 0; i < 16; ++i) s[nb][i] -= sl2 * fabsf(d + (float)(16 * (i >> 3) + (i & 7)));
      }
      if constexpr (MASK && MK != 0) {
        // Key t0 + 16 (i >> 3) + 8 hh + (i & 7) is visible iff its offset
        // 16 (i >> 3) + (i & 7) from t0 + 8 hh lies in one of the row's ranges.
        const int base = st * 32 + 8 * hh;
        const int a1 = mr[nb][0] - base, b1 = mr[nb][1] - base, a2 = mr[nb][2] - base, b2 = mr[nb][3] - base;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int o = 16 * (i >> 3) + (i & 7);
          if (!((o >= a1 && o <= b1) || (o >= a2 && o <= b2))) s[nb][i] = -INFINITY;
        }
      } else if constexpr (MASK) {
        // Key t0 + 16 (i >> 3) + 8 hh + (i & 7) is visible iff its offset
        // 16 (i >> 3) + (i & 7) (an inline constant) <= lim.
        const int t0 = st * 32, qa = wq0 + 32 * nb + l32 + off;
        int lim = r.k_len - 1 - t0;
        if (CAUSAL) lim = min(lim, qa - t0);
        else if (WR >= 0) lim = min(lim, qa + WR - t0);
        lim -= 8 * hh;
        // ... and >= lo (left window).
        const int lo = WL >= 0 ? qa - WL - t0 - 8 * hh : INT_MIN;
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (16 * (i >> 3) + (i & 7) > lim || 16 * (i >> 3) + (i & 7) < lo) s[nb][i] = -INFINITY;
      }
      float mx = fmaxf(s[nb][0], s[nb][1]);
#pragma unroll
      for (int i = 2; i < 16; ++i) mx = fmaxf(mx, s[nb][i]);
      mx = max_hh(mx);
      const float cand = CAP ? mx : mx * c_scale;
      const bool need = commit && cand > m_run[nb] + PF_RESCALE;
      f[nb] = need ? fast_exp2(m_run[nb] - cand) : 1.0f;
      m_run[nb] = need ? cand : m_run[nb];
      l_run[nb] *= f[nb];
    }
  };
  // Phase B: probabilities (<= 2^8), row sums, packed B operand of O^T.
  // The row sums add the fp32 probabilities: summing the 16-bit values that
  // P.V consumes (v_dot2 with (1, 1), half the instructions) puts the LSE
  // ~1.5e-3 off for bf16, past its 1e-4 bar.
  auto phase_b = [&](f32x16 (&s)[NB], u32x4 (&pop)[NB][2]) {
    const float sc = CAP ? 1.0f : c_scale;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const float mref = m_run[nb] == -INFINITY ? 0.0f : m_run[nb];
      float psum = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = fast_exp2(fmaf(s[nb][i], sc, -mref));
        s[nb][i] = p;
        psum += p;
      }
      l_run[nb] += psum;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        u32x4 w;
#pragma unroll
        for (int q = 0; q < 4; ++q) w[q] = pack2<T>(s[nb][8 * c + 2 * q], s[nb][8 * c + 2 * q + 1]);
        pop[nb][c] = w;
      }
    }
  };
  auto pv = [&](int st, const u32x4 (&pop)[NB][2], auto par) {
    constexpr int PAR = decltype(par)::value;
    const char* vl;
    if constexpr (PAR < 0) vl = vbuf0 + ((st >> 1) & 1) * VTILE + (st & 1) * 32 * 64;
    else vl = vbuf0 + (PAR >> 1) * VTILE + (PAR & 1) * 32 * 64;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int imm = 16 * c * 64 + db * PF_VBLOCK_BYTES;
        const u32x2 lo = lds_read_tr(vl, vrd + imm);
        const u32x2 hi = lds_read_tr(vl, vrd + imm + 4 * 64);
        const u32x4 av = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) o[nb][db] = mfma32<T>(av, pop[nb][c], o[nb][db]);
      }
  };
  const std::integral_constant<int, -1> at_run_time;
  auto rescale_o = [&](const float (&f)[NB]) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (__builtin_expect(__any(f[nb] != 1.0f), 0)) {
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[nb][db][i] *= f[nb];
      }
    }
  };

  // One pipeline stage: P(st) from S(st), S(st+1), O += V P(st), phase A of
  // S(st+1); f carries O's pending rescale factors.
  //
  // LDS traffic, at the start of tile j (even stages): wait for this wave's
  // DMAs and barrier, after which V(j), K(j) rows 32..63 and K(j+1) rows
  // 0..31 are resident and every wave is done with V(j-1), K(j-1) rows
  // 32..63 and K(j) rows 0..31; then V(j+1), K(j+1) rows 32..63 and K(j+2)
  // rows 0..31 are issued into the freed buffer halves.  With a full mode
  // true the caller guarantees that those tiles lie inside the request.
  // FP8: the staging tile holds tile j+1; it is widened into buffer
  // (j+1) & 1 (free since tile j-1 is done), then refilled with tile j+2.
  auto tile_start = [&](auto mode, int st) {
    if ((st & 1) == 0) {
      const int j = st >> 1;
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
      if constexpr (FQ) {
        // V(j+1) is in staging slot (j+1) % 2 and buffer (j+1) % 2 is free
        // (V(j-1) is done); slot j % 2 was widened a tile ago, so it takes
        // V(j+2).  K as in the 16-bit path.
        if (j + 1 < n_tiles) widen_v((j + 1) & 1, (j + 1) & 1);
        if (j + 2 < n_tiles) dma_v8(j + 2, j & 1);
        if (j + 1 < n_tiles) dma_k(mode, j + 1, (j + 1) & 1, 1);
        if (j + 2 < n_tiles) dma_k(mode, j + 2, j & 1, 0);
      } else if constexpr (FP8) {
        if (j + 1 < n_tiles) {
          widen_tile((j + 1) & 1);
          __syncthreads();
          if (j + 2 < n_tiles) dma_fp8(j + 2);
        }
      } else {
        if (j + 1 < n_tiles) {
          dma_v(mode, j + 1, (j + 1) & 1);
          dma_k(mode, j + 1, (j + 1) & 1, 1);
        }
        if (j + 2 < n_tiles) dma_k(mode, j + 2, j & 1, 0);
      }
    }
  };
  // Tiles j + 1 and (if it exists) j + 2 hold 64 keys of the request each.
  auto dma_full = [&](int j) { return PF_BN * (j + 2 < n_tiles ? j + 3 : j + 2) <= r.k_len; };
  // Steady state: stage st and st+1 both active, st+1 unmasked.  One
  // straight scheduling region: phase B(st) under the MFMAs of S(st+1),
  // phase A(st+1) under the MFMAs of P.V(st).
  // par: stage st's parities, as for qk / pv.
  auto step_hot = [&](auto mode, auto par, int st, f32x16 (&sc)[NB], f32x16 (&sn)[NB], float (&f)[NB])
                      __attribute__((always_inline)) {
    tile_start(mode, st);
    rescale_o(f);
    u32x4 pop[NB][2];
    phase_b(sc, pop);
    constexpr int PAR = decltype(par)::value;
    if constexpr (PAR < 0) {
      qk(st + 1, sn, at_run_time);
    } else {
      // stage st + 1: the other half, in the next buffer after a second half
      constexpr int P = PAR >> 1, E = PAR & 1;
      qk(st + 1, sn, std::integral_constant<int, 2 * (E ? P ^ 1 : P) + (E ^ 1)>());
    }
    pv(st, pop, par);
    if constexpr (!CAP) {
      // Phase A proper (the row max across the lane pair, the rescale factor,
      // the running max and sum) runs only when some lane holds a score past
      // the rescale threshold or has no running max yet; otherwise it would
      // leave the state as it is (+2% on config 2).
      bool over = false;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        float mx = fmaxf(sn[nb][0], sn[nb][1]);
#pragma unroll
        for (int i = 2; i < 16; ++i) mx = fmaxf(mx, sn[nb][i]);
        over |= !(mx * c_scale <= m_run[nb] + PF_RESCALE);
      }
      if (__builtin_expect(__any(over), 0)) {
        phase_a(std::integral_constant<bool, false>(), st + 1, sn, true, f);
      } else {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) f[nb] = 1.0f;
      }
    } else {
      phase_a(std::integral_constant<bool, false>(), st + 1, sn, true, f);
    }
    // Scheduling strategy of the AMDGPU backend that interleaves LDS reads
    // with the MFMAs (the default schedule issues each K operand read one
    // MFMA ahead): +1-2.5% on config 2, measured on two boxes; hand-written
    // group patterns (sched_group_barrier) measured 7% slower.
    if constexpr (!FP8) __builtin_amdgcn_iglp_opt(0);
  };
  // Any stage: inactive waves only keep the barrier cadence; S(st+1) is
  // computed even when stage st+1 lies past this wave's causal range (its K
  // rows hold valid or stale finite data) and its phase A then commits
  // nothing.
  // With windows, a wave inactive at st (left of its window) but active at
  // st+1 only computes S(st+1).
  auto step_any = [&](int st, f32x16 (&sc)[NB], f32x16 (&sn)[NB], float (&f)[NB]) {
    tile_start(std::integral_constant<int, PF_ANY_TILE>(), st);
    const bool act = active(st), act_n = st + 1 < n_stages && active(st + 1);
    u32x4 pop[NB][2];
    if constexpr (GEN) {
      if (!act && !act_n) return;
      if (act) {
        rescale_o(f);
        phase_b(sc, pop);
      }
      qk(st + 1, sn, at_run_time);
      if (act) pv(st, pop, at_run_time);
    } else {
      if (!act) return;
      rescale_o(f);
      phase_b(sc, pop);
      qk(st + 1, sn, at_run_time);
      pv(st, pop, at_run_time);
    }
    if (needs_mask(st + 1)) phase_a(std::integral_constant<bool, true>(), st + 1, sn, act_n, f);
    else phase_a(std::integral_constant<bool, false>(), st + 1, sn, act_n, f);
  };
  auto hot = [&](int st) { return st < n_stages && active(st) && !needs_mask(st); };

  // The key pipeline over tiles tile0 .. n_tiles - 1 (stages st0 .. n_stages - 1).
  auto run_keys = [&]() {
  if (st0 < n_stages) {
    // Prologue: tile tile0 and K(tile0 + 1) rows 0..31 in LDS; S(st0) and
    // its phase A.
    const std::integral_constant<int, PF_ANY_TILE> any_tile;
    if constexpr (FQ) {
      dma_k(any_tile, tile0, tile0 & 1, 0);
      dma_k(any_tile, tile0, tile0 & 1, 1);
      dma_v8(tile0, tile0 & 1);
      if (tile0 + 1 < n_tiles) {
        dma_k(any_tile, tile0 + 1, (tile0 + 1) & 1, 0);
        dma_v8(tile0 + 1, (tile0 + 1) & 1);
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
      widen_v(tile0 & 1, tile0 & 1);   // visible after the barrier that starts the first tile
    } else if constexpr (FP8) {
      dma_fp8(tile0);
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
      widen_tile(tile0 & 1);
      __syncthreads();
      if (tile0 + 1 < n_tiles) dma_fp8(tile0 + 1);
    } else {
      dma_k(any_tile, tile0, tile0 & 1, 0);
      dma_k(any_tile, tile0, tile0 & 1, 1);
      dma_v(any_tile, tile0, tile0 & 1);
      if (tile0 + 1 < n_tiles) dma_k(any_tile, tile0 + 1, (tile0 + 1) & 1, 0);
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
    }
    f32x16 sa[NB], sb[NB];
    float f[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) f[nb] = 1.0f;
    if (active(st0)) {
      qk(st0, sa, at_run_time);
      phase_a(std::integral_constant<bool, true>(), st0, sa, true, f);
    }
    // Even stage st holds S in sa, odd in sb.  The unmasked two-stage loop
    // runs first; with windows it is re-entered at even stages where this
    // wave is active (its window may start after st0).
    // The hot loop is instantiated once per K/V layout (packed, paged).
    int st = st0;
    if constexpr (GEN) {
      auto run_hot = [&](auto mode) {
        const std::integral_constant<int, -1> rt;
        for (; hot(st + 1) && hot(st + 2) && dma_full(st >> 1); st += 2) {
          step_hot(mode, rt, st, sa, sb, f);
          step_hot(mode, rt, st + 1, sb, sa, f);
        }
      };
      while (st < n_stages) {
        if (!(st & 1) && active(st)) {
          if (paged) run_hot(std::integral_constant<int, PF_FULL_PAGED>());
          else run_hot(std::integral_constant<int, PF_FULL_PACKED>());
        }
        if (st >= n_stages) break;
        if (st & 1) step_any(st, sb, sa, f);
        else step_any(st, sa, sb, f);
        ++st;
      }
    } else {
      // Closed form of hot(st + 1) && hot(st + 2) && dma_full(st / 2) for
      // even st >= st0 without windows: hot(s) <=> wave_rows && s < hb, and
      // dma_full(j) <=> j <= jmax (both conditions are prefixes of the
      // stage / tile range).
      const int kf = r.k_len / PF_BN;
      const int jmax = n_tiles <= kf ? kf - 2 : kf - 3;
      int hb = min(n_stages, r.k_len / 32);
      if constexpr (CAUSAL) hb = min(hb, max(wave_qabs_lo + 1, 0) / 32);
      const int lim = wave_rows ? min(hb - 2, 2 * jmax + 1) : INT_MIN;
      // 64-dim 16-bit tiles: two tiles per iteration, so every stage's K/V
      // buffer and half are constants (immediate LDS offsets instead of a
      // VALU add per operand address): one loop per buffer of the first
      // tile, then the last odd tile with run-time parities.  Same process
      // on config 2's lengths at 32/8 heads: causal 770 -> 812 TFLOP/s.  The
      // 128-dim tile ran 5.5-6.5% slower that way (config 2 948 -> 896,
      // non-causal 1078 -> 1005, with 5 fewer VALU instructions per stage),
      // so the other tiles keep one tile per iteration (E4M3 K/V also need
      // their staging refill addresses scalar).
      auto run_hot = [&](auto mode) {
        const std::integral_constant<int, -1> rt;
        if constexpr (FP8 || DQ != 64) {
          for (; st < lim; st += 2) {
            step_hot(mode, rt, st, sa, sb, f);
            step_hot(mode, rt, st + 1, sb, sa, f);
          }
        } else {
          auto two_tiles = [&](auto p0, auto p1) {
            for (; st + 2 < lim; st += 4) {
              step_hot(mode, std::integral_constant<int, 2 * decltype(p0)::value>(), st, sa, sb, f);
              step_hot(mode, std::integral_constant<int, 2 * decltype(p0)::value + 1>(), st + 1, sb, sa, f);
              step_hot(mode, std::integral_constant<int, 2 * decltype(p1)::value>(), st + 2, sa, sb, f);
              step_hot(mode, std::integral_constant<int, 2 * decltype(p1)::value + 1>(), st + 3, sb, sa, f);
            }
          };
          if (((st >> 1) & 1) == 0) two_tiles(std::integral_constant<int, 0>(), std::integral_constant<int, 1>());
          else two_tiles(std::integral_constant<int, 1>(), std::integral_constant<int, 0>());
          if (st < lim) {
            step_hot(mode, rt, st, sa, sb, f);
            step_hot(mode, rt, st + 1, sb, sa, f);
            st += 2;
          }
        }
      };
      if (active(st)) {
        if (paged) run_hot(std::integral_constant<int, PF_FULL_PAGED>());
        else run_hot(std::integral_constant<int, PF_FULL_PACKED>());
      }
      for (; st < n_stages; ++st) {
        if (st & 1) step_any(st, sb, sa, f);
        else step_any(st, sa, sb, f);
      }
    }
  }
  };
  if constexpr (MK == 2) {
    if (mk_split) {
      // The prefix's tiles, then those of the windows; the running (m, l, O)
      // carry over, and a barrier keeps the second run's first DMAs off tiles
      // still being read.
      const int kv_all = kv_end;
      set_ranges(1);
      wave_bounds();
      kv_end = min(mk_p, kv_all);
      n_tiles = (kv_end + PF_BN - 1) / PF_BN, n_stages = (kv_end + 31) / 32;
      tile0 = 0, st0 = 0;
      run_keys();
      __syncthreads();
      set_ranges(2);
      wave_bounds();
      kv_end = kv_all;
      n_tiles = (kv_end + PF_BN - 1) / PF_BN, n_stages = (kv_end + 31) / 32;
      tile0 = max(qa_first - mk_w + 1, 0) / PF_BN, st0 = 2 * tile0;
      run_keys();
    } else {
      set_ranges(0);
      wave_bounds();
      run_keys();
    }
  } else {
    if constexpr (MK == 1) {
      set_ranges(0);
      wave_bounds();
    }
    run_keys();
  }

  // Epilogue: O = O^T / l, LSE = m * ln2 + ln(l).
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const float lt = sum_hh(l_run[nb]);
    const int row = wq0 + 32 * nb + l32;
    if (row < r.q_len) {
      const float inv = lt > 0.0f ? vdsc / lt : 0.0f;
      const int64_t tq = (int64_t)r.q_begin + row;
      uint16_t* op = (uint16_t*)a.out + tq * a.out_stride[0] + (int64_t)h * a.out_stride[1] + (TWO_PARTS ? vpart * DVT : 0) + 4 * hh;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          if (32 * db + 8 * g + 8 > DVT) continue;   // padding columns
          uint2 w;
          w.x = pack2<T>(o[nb][db][4 * g] * inv, o[nb][db][4 * g + 1] * inv);
          w.y = pack2<T>(o[nb][db][4 * g + 2] * inv, o[nb][db][4 * g + 3] * inv);
          *(uint2*)(op + 32 * db + 8 * g) = w;
        }
      if (hh == 0 && (!TWO_PARTS || vpart == 0))
        a.lse[(int64_t)h * a.lse_stride[0] + tq * a.lse_stride[1]] = lt > 0.0f ? m_run[nb] * LN2 + logf(lt) : -INFINITY;
    }
  }
}

// Waves per workgroup, 32-row query blocks per wave and workgroups per CU
// per head-dim pair (LDS holds two K and two V tiles per workgroup).
#ifndef FA_PF128_W
#define FA_PF128_W 4
#define FA_PF128_NB 1
#define FA_PF128_MINB 2
#endif
template <int DQ, int DV> struct PrefillTile;
// 64/64: three workgroups per CU (+6-10% over two on config 2's lengths,
// +9% with softcap); its window variant spills at that register budget and
// keeps two (MINB_WIN).
template <> struct PrefillTile<64, 64> { static constexpr int W = 4, NB = 1, MINB = 3, MINB_WIN = 2; };
template <> struct PrefillTile<128, 128> {
  static constexpr int W = FA_PF128_W, NB = FA_PF128_NB, MINB = FA_PF128_MINB, MINB_WIN = MINB;
};
// 192/128: two workgroups per CU (2 x 80 KiB of LDS) trade registers for a
// second wave per SIMD, at every grid size (one workgroup per CU ran 7-48%
// slower even on 128-workgroup launches).
template <> struct PrefillTile<192, 128> { static constexpr int W = 4, NB = 1, MINB = 2, MINB_WIN = 2; };
// 256/256 (the softcap routes of pick_256): one wave per SIMD (128 KiB of LDS).
template <> struct PrefillTile<256, 256> { static constexpr int W = 4, NB = 1, MINB = 1, MINB_WIN = 1; };
// 256-dim 16-bit heads run as two 256/128 halves of V (prefill_vparts): eight
// waves in 96 KiB of LDS, two per SIMD.
template <> struct PrefillTile<256, 128> { static constexpr int W = 8, NB = 1, MINB = 1, MINB_WIN = 1; };

template <int DQ, int DV>
constexpr size_t lds_bytes() {
  return 2 * (size_t)(DQ / 64 + DV / 64) * PF_GROUP_BYTES;
}

using PrefillKernel = void (*)(fa_attn_args, PrefillShape);

struct PrefillChoice {
  PrefillKernel kern;
  int bm, threads;
  size_t lds;
  int vparts;   // workgroups per work item, one per DV-column part of the head (prefill_vparts)
};

// score: 0 plain, 1 softcap, 2 ALiBi, 3 softcap then ALiBi; mk: vLLM
// mask kind (0 none; instantiated for unpadded head dims without ALiBi, not
// for the one-pass E4M3 256/256 tile: E4M3 d256 masks run as V halves).
template <typename T, int DQ, int DV, bool CAUSAL, typename S, int DQT, int DVT, typename KT>
PrefillChoice pick_tile(int score, bool win, int mk) {
  PrefillChoice c;
  const bool cap = score == 1;
  if (mk != 0) {
    if constexpr (CAUSAL || DQT != DQ || DVT != DV || (KT::id == FA_E4M3 && DV == 256)) {
      return PrefillChoice{nullptr, 0, 0, 0};
    } else {
      if (score == 2) return PrefillChoice{nullptr, 0, 0, 0};
      if (mk == 1)
        c.kern = cap ? prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB_WIN, false, true, false, DQT, DVT, KT, false, T, 1>
                     : prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB_WIN, false, false, false, DQT, DVT, KT, false, T, 1>;
      else
        c.kern = cap ? prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB_WIN, false, true, false, DQT, DVT, KT, false, T, 2>
                     : prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB_WIN, false, false, false, DQT, DVT, KT, false, T, 2>;
    }
  } else if (score >= 2) {   // ALiBi (3: after a softcap)
    // With windows, softcap or E4M3 K/V: unpadded 64 / 128 / 256-dim heads
    // (E4M3 K/V at d256 on the V-half tile only).
    constexpr bool MORE = DQT == DQ && DVT == DV &&
                          ((DQ == DV && (DQ == 64 || DQ == 128 || DQ == 256)) || (DQ == 256 && DV == 128)) &&
                          !(KT::id == FA_E4M3 && DV == 256);
    const bool capa = score == 3;
    if (!capa && !win && KT::id != FA_E4M3) {
      c.kern = prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB, CAUSAL, false, false, DQT, DVT, KT, true>;
    } else {
      if constexpr (!MORE) {
        return PrefillChoice{nullptr, 0, 0, 0};
      } else {
        if (win)
          c.kern = capa ? prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB_WIN, CAUSAL, true, true, DQT, DVT, KT, true>
                        : prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB_WIN, CAUSAL, false, true, DQT, DVT, KT, true>;
        else
          c.kern = capa ? prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB, CAUSAL, true, false, DQT, DVT, KT, true>
                        : prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB, CAUSAL, false, false, DQT, DVT, KT, true>;
      }
    }
  } else if (win)
    c.kern = cap ? prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB_WIN, CAUSAL, true, true, DQT, DVT, KT>
                 : prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB_WIN, CAUSAL, false, true, DQT, DVT, KT>;
  else
    c.kern = cap ? prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB, CAUSAL, true, false, DQT, DVT, KT>
                 : prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB, CAUSAL, false, false, DQT, DVT, KT>;
  c.bm = 32 * S::NB * S::W;
  c.threads = 64 * S::W;
  c.lds = lds_bytes<DQ, DV>() + (KT::id == FA_E4M3 ? 64 * (size_t)(DQ + DV) : 0);   // + FP8 staging tile
  c.vparts = prefill_vparts<DQ, DV>();
  return c;
}

// (DQ, DV) = the tile; (DQT, DVT) = the tensors' head dims padded into it;
// KT = the K/V storage type.
template <typename T, typename KT, int DQ, int DV, int DQT = DQ, int DVT = DV>
PrefillChoice pick(bool causal, int score, bool win, int mk) {
  // Mask kinds carry their own causality: the non-causal instances take them.
  return causal && mk == 0 ? pick_tile<T, DQ, DV, true, PrefillTile<DQ, DV>, DQT, DVT, KT>(score, win, mk)
                           : pick_tile<T, DQ, DV, false, PrefillTile<DQ, DV>, DQT, DVT, KT>(score, win, mk);
}

// Head dims of the reference's fast path (flash_attn_mps/_attention.py:149-158:
// 32, 64, 72, 80, 96, 128, 256) plus DIFFKV 192/128; 32 runs in the 64-dim
// tile and 72/80/96 in the 128-dim tile.  FP8 K/V: 64, 128, 256.  The
// variants are split over four translation units (prefill_inst_*.hip), by
// query dtype and by head dim (16-bit K/V up to 128 / the rest), so that
// they compile in parallel.
template <typename T>
PrefillChoice pick_dims_small(int64_t dq, int64_t dv, bool causal, int score, bool win, int mk) {
  if (dq != dv) return PrefillChoice{nullptr, 0, 0, 0};
  switch (dq) {
    case 32: return pick<T, T, 64, 64, 32, 32>(causal, score, win, mk);
    case 64: return pick<T, T, 64, 64>(causal, score, win, mk);
    case 72: return pick<T, T, 128, 128, 72, 72>(causal, score, win, mk);
    case 80: return pick<T, T, 128, 128, 80, 80>(causal, score, win, mk);
    case 96: return pick<T, T, 128, 128, 96, 96>(causal, score, win, mk);
    case 128: return pick<T, T, 128, 128>(causal, score, win, mk);
    default: return PrefillChoice{nullptr, 0, 0, 0};
  }
}

// 256-dim heads: two V-column halves per work item (prefill_vparts),
// each an eight-wave 256/128 tile at two waves per SIMD (the one-pass
// 256/256 tile holds four waves, one per SIMD, and spills more).  The halves
// recompute S, with every tanh of a softcap: 16-bit softcaps, and E4M3
// softcaps with a window and no ALiBi, keep the one-pass tile (which has no
// E4M3 ALiBi instance).  Measured on config 2's
// lengths at 16/8 heads (TFLOP/s, one-pass -> halves): bf16 causal 456 ->
// 597, non-causal 629 -> 716, ALiBi 404 -> 519, left window 1023 260 -> 292,
// vLLM mm_prefix +36%, rswa +8%, softcap 50 560 -> 519, softcap + window
// 346 -> 257; E4M3 K/V causal 299 -> 564, non-causal 342 -> 657, softcap
// 339 -> 444, window 221 -> 255, softcap + window 285 -> 228.
template <typename T, typename KT>
PrefillChoice pick_256(bool causal, int score, bool win, int mk) {
  const bool cap = score == 1 || score == 3;
  if (cap && (KT::id != FA_E4M3 || (win && score == 1))) return pick<T, KT, 256, 256>(causal, score, win, mk);
  return pick<T, KT, 256, 128>(causal, score, win, mk);
}

template <typename T>
PrefillChoice pick_dims_large(int64_t dq, int64_t dv, bool causal, int score, bool win, bool fp8, int mk) {
  if (fp8) {
    if (dq != dv) return PrefillChoice{nullptr, 0, 0, 0};
    switch (dq) {
      case 64: return pick<T, E4M3T, 64, 64>(causal, score, win, mk);
      case 128: return pick<T, E4M3T, 128, 128>(causal, score, win, mk);
      case 256: return pick_256<T, E4M3T>(causal, score, win, mk);
      default: return PrefillChoice{nullptr, 0, 0, 0};
    }
  }
  if (dq == 192 && dv == 128) return pick<T, T, 192, 128>(causal, score, win, mk);
  if (dq == 256 && dv == 256) return pick_256<T, T>(causal, score, win, mk);
  return PrefillChoice{nullptr, 0, 0, 0};
}

// E4M3 queries over E4M3 K/V (S on the FP8 MFMA), output type T; head dims
// 64, 128 and 256 (256 as two 256/128 V-column halves, every variant: on
// config 2's lengths at 16/8 heads, one pass -> halves, TFLOP/s: causal 617
// -> 828, non-causal 715 -> 965, softcap 50 589 -> 655, left window 1023
// 357 -> 618, softcap + window 415 -> 441).  K tiles hold raw bytes
// (ceil(DQ / 128) column groups), V is staged twice (64 x DV bytes each) and
// widened into 16-bit tiles.
template <typename T, int DQ, int DV, bool CAUSAL>
PrefillChoice pick_tile_fp8q(int score, bool win) {
  using S = PrefillTile<DQ, DV>;
  if (score >= 2) return PrefillChoice{nullptr, 0, 0, 0};   // ALiBi with E4M3 queries: the generic kernel
  const bool cap = score == 1;
  PrefillChoice c;
  if (win)
    c.kern = cap ? prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB_WIN, CAUSAL, true, true, DQ, DV, E4M3T, false, E4M3T>
                 : prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB_WIN, CAUSAL, false, true, DQ, DV, E4M3T, false, E4M3T>;
  else
    c.kern = cap ? prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB, CAUSAL, true, false, DQ, DV, E4M3T, false, E4M3T>
                 : prefill_kernel<T, DQ, DV, S::W, S::NB, S::MINB, CAUSAL, false, false, DQ, DV, E4M3T, false, E4M3T>;
  c.bm = 32 * S::NB * S::W;
  c.threads = 64 * S::W;
  c.lds = 2 * (size_t)((DQ + 127) / 128) * PF_GROUP_BYTES + 2 * (size_t)(DV / 64) * PF_GROUP_BYTES + 2 * 64 * (size_t)DV;
  c.vparts = prefill_vparts<DQ, DV>();
  return c;
}

template <typename T>
PrefillChoice pick_dims_fp8q(int64_t dq, int64_t dv, bool causal, int score, bool win) {
  if (dq != dv) return PrefillChoice{nullptr, 0, 0, 0};
  if (dq == 64) return causal ? pick_tile_fp8q<T, 64, 64, true>(score, win) : pick_tile_fp8q<T, 64, 64, false>(score, win);
  if (dq == 128)
    return causal ? pick_tile_fp8q<T, 128, 128, true>(score, win) : pick_tile_fp8q<T, 128, 128, false>(score, win);
  if (dq == 256)
    return causal ? pick_tile_fp8q<T, 256, 128, true>(score, win) : pick_tile_fp8q<T, 256, 128, false>(score, win);
  return PrefillChoice{nullptr, 0, 0, 0};
}

// Defined in prefill_inst_{bf16,f16}_{small,large}.hip and prefill_inst_fp8q.hip.
PrefillChoice pick_bf16_small(int64_t dq, int64_t dv, bool causal, int score, bool win, int mk);
PrefillChoice pick_f16_small(int64_t dq, int64_t dv, bool causal, int score, bool win, int mk);
PrefillChoice pick_bf16_large(int64_t dq, int64_t dv, bool causal, int score, bool win, bool fp8, int mk);
PrefillChoice pick_f16_large(int64_t dq, int64_t dv, bool causal, int score, bool win, bool fp8, int mk);
PrefillChoice pick_fp8q(int out_dtype, int64_t dq, int64_t dv, bool causal, int score, bool win);

}  // namespace fa_prefill

#endif  // FA_PREFILL_KERNEL_H
