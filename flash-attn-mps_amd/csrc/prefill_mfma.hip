// MFMA FlashAttention prefill for gfx950 (bf16 / fp16, Dqk = Dv in {64, 128, 256}).
//
// Semantics follow the reference's fast path (flash_attn_mps/_attention.py:149-158,
// flash_attn_mps/kernels/attention_fast.metal:103-597): packed or paged K/V, GQA,
// lower-right causality, optional softcap, fp32 softmax and LSE.
//
// gfx950 design
// * A workgroup is 4 waves; each wave owns NB x 32 query rows of one head, so a
//   workgroup covers BM = 128 * NB rows.  K/V tiles of BN = 64 keys are staged
//   in LDS (double buffered; the next tile's global loads are issued before the
//   current tile's MFMAs).
// * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16
//   (A = K rows from LDS, B = Q^T held in registers for the whole kernel).  A
//   lane then holds 32 keys of ONE query column, so the row max / row sum of
//   the softmax are in-lane reductions plus one exchange with lane ^ 32.
// * K rows are stored in LDS at row sigma(r) (bits 2 and 3 of r swapped) so
//   that, in the score layout, every lane's 8 consecutive accumulator values
//   are 8 consecutive keys.  Those 8 probabilities, rounded to bf16/fp16, are
//   directly the B operand of O^T += V^T P^T; V is written transposed into LDS
//   (V^T rows = head dims) so its A operand is one 16-byte LDS read.
// * exp2 with softmax_scale*log2(e) folded into one FMA; the running max is
//   only moved (and O rescaled) when a tile raises it by more than 2^8, which
//   keeps probabilities <= 256 and skips almost all rescales.
// * Work is ordered per XCD: each XCD runs whole (request, KV head) pairs one
//   after another, query blocks heaviest-first within a pair (the causal
//   triangle makes late blocks the longest), so resident workgroups share K/V
//   in their XCD's L2.  K/V tiles are read with bounded buffer loads.
#include "attn_common.h"

namespace {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

constexpr int PF_WAVES = 4;
constexpr int PF_THREADS = 64 * PF_WAVES;
constexpr float PF_RESCALE = 8.0f; // log2 headroom before the running max moves

// Tile shape for head dims <= 128: NB 32-row query blocks per wave, KT
// 32-key blocks per K/V tile, MINB workgroups per CU in the launch bounds.
#ifndef FA_PF_NB
#define FA_PF_NB 1
#endif
#ifndef FA_PF_KT
#define FA_PF_KT 2
#endif
#ifndef FA_PF_MINB
#define FA_PF_MINB 2
#endif

template <typename T> FA_DEV f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);
template <> FA_DEV f32x16 mfma32<BF16T>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <> FA_DEV f32x16 mfma32<F16T>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
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

// Swap bits 2 and 3 of a row index (an involution).
FA_DEV int sigma(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

struct PrefillShape {
  int n_qblocks;
  int log2_page;   // paged K/V: page size = 1 << log2_page
};

template <typename T, int D, int NB, int KT, int MINB, bool CAUSAL>
__global__ __launch_bounds__(PF_THREADS, MINB) void prefill_kernel(const fa_attn_args a, const PrefillShape shp) {
  constexpr int BM = PF_WAVES * NB * 32;
  constexpr int BN = 32 * KT;
  constexpr int KST = D / 16;                  // k-steps of the QK^T MFMA
  constexpr int DB = D / 32;                   // 32-row blocks of O^T
  constexpr int KLD = D + 8;                   // LDS row stride of K (elements)
  constexpr int VLD = BN + 8;                  // LDS row stride of V^T
  constexpr int KTILE = BN * KLD, VTILE = D * VLD;
  constexpr int KCH = BN * D / 8 / PF_THREADS; // 16-byte K chunks per thread
  constexpr int VUNITS = (BN / 4) * (D / 8);   // (4 keys x 8 dims) V units per tile
  constexpr int VPT = (VUNITS + PF_THREADS - 1) / PF_THREADS;
  static_assert(KCH >= 1 && BN * D / 8 % PF_THREADS == 0, "K staging shape");

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  // Work order.  Workgroups are dispatched round-robin over the 8 XCDs
  // (XCD = blockIdx % 8), each with its own L2.  XCD x takes the (request,
  // KV head) pairs p = x, x + 8, ... one after another, and within a pair the
  // query blocks of its G query heads heaviest-first, so the workgroups
  // resident on an XCD at any time share one pair's K/V in that XCD's L2.
  const int G = (int)(a.heads_q / a.heads_k);
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
  const int per_pair = shp.n_qblocks * G;
  const int64_t pair = (int64_t)(slot / per_pair) * 8 + xcd;
  if (pair >= a.batch * a.heads_k) return;
  const int rem = slot % per_pair;
  const int qb = shp.n_qblocks - 1 - rem / G;
  const int64_t b = pair / a.heads_k;
  const int h = (int)(pair % a.heads_k) * G + rem % G;
  const RequestInfo r = load_request(a, b);
  const int q0 = qb * BM;
  if (q0 >= r.q_len) return;
  const int kh = h / (int)(a.heads_q / a.heads_k);
  const int off = r.k_len - r.q_len;   // absolute position of query row i is i + off
  int kv_end = r.k_len;
  if (CAUSAL) kv_end = min(kv_end, min(q0 + BM, r.q_len) - 1 + off + 1);
  const int n_tiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;

  const T* __restrict__ Q = (const T*)nullptr;
  (void)Q;
  const uint16_t* qg = (const uint16_t*)a.q;
  const uint16_t* kg = (const uint16_t*)a.k;
  const uint16_t* vg = (const uint16_t*)a.v;

  // Q^T operand for the whole kernel: lane holds Q[row][16kk + 8hh .. +8].
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);   // wave index as a scalar
  const int wq0 = q0 + wave_u * NB * 32;
  u32x4 qop[NB][KST];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int row = wq0 + nb * 32 + l32;
    const bool ok = row < r.q_len;
    const uint16_t* qp = qg + ((int64_t)r.q_begin + row) * a.q_stride[0] + (int64_t)h * a.q_stride[1] + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < KST; ++kk) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (ok) v = *(const u32x4*)(qp + 16 * kk);
      qop[nb][kk] = v;
    }
  }
  // Complete the Q loads here: otherwise the loop header cannot prove them
  // done and every iteration would wait for all in-flight K/V loads before
  // its first MFMA (s_waitcnt vmcnt(0); expcnt/lgkmcnt left unconstrained).
  __builtin_amdgcn_s_waitcnt(0x0F70);

  const bool paged = a.page_size != 0;
  const int lp = shp.log2_page;
  // Storage offset (elements) of key `key`; used per lane only when a wave's
  // rows can span two 16-key groups (D = 64).
  auto row_offset = [&](const int64_t* st, int key) -> int64_t {
    if (paged) {
      const int page = key >> lp;
      const int64_t blk = a.block_table[b * a.bt_stride[0] + (int64_t)page * a.bt_stride[1]];
      return blk * st[0] + (int64_t)(key - (page << lp)) * st[1] + (int64_t)kh * st[2];
    }
    return ((int64_t)r.k_base + key) * st[1] + (int64_t)kh * st[2];
  };

  // Staging layout.  K: 16-byte chunk c of a thread covers row r0 + lane/(D/8)
  // (r0 uniform per wave) and columns 8*(lane % (D/8)).  V: unit u of a thread
  // covers 4 keys x 8 dims with the dims fastest across lanes (coalesced
  // global reads).  For D >= 128 every wave's rows of a chunk/unit lie inside
  // one 16-key group, whose storage base is wave-uniform (one scalar block
  // table read per group and tile); lanes add a 32-bit offset computed once.
  constexpr int KROWS_W = 64 / (D / 8);
  constexpr int VROWS_W = 4 * 64 / (D / 8);
  constexpr bool UNIFORM = VROWS_W <= 16;
  int kgrp[KCH], koff[KCH], kst[KCH];
#pragma unroll
  for (int c = 0; c < KCH; ++c) {
    const int r0 = (64 * wave_u + PF_THREADS * c) / (D / 8);
    const int row = r0 + lane / (D / 8), col8 = lane % (D / 8);
    kgrp[c] = r0 & ~15;
    koff[c] = 2 * ((row - kgrp[c]) * (int)a.k_stride[1] + col8 * 8);   // bytes
    kst[c] = sigma(row) * KLD + col8 * 8;
  }
  int vgrp[VPT], voff[VPT][4], vst[VPT];
  bool vunit[VPT];
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const int uid0 = 64 * wave_u + PF_THREADS * u;
    const int uid = uid0 + lane;
    const int kgp = uid / (D / 8), dc = uid % (D / 8);
    vunit[u] = uid < VUNITS;
    vgrp[u] = (4 * (uid0 / (D / 8))) & ~15;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) voff[u][rr] = 2 * ((4 * kgp + rr - vgrp[u]) * (int)a.v_stride[1] + dc * 8);
    // V^T element (dim, key) lives at dim*VLD + 8*((key/8) ^ ((dim/16) & 7)) + key%8:
    // with 64 LDS banks, 32 lanes writing 8 bytes (dims 8*dc + d, two key
    // groups) and 16 lanes reading 16 bytes (16 consecutive dims) both hit
    // distinct banks.
    vst[u] = 8 * dc * VLD + 8 * ((kgp >> 1) ^ ((dc >> 1) & 7)) + 4 * (kgp & 1);
  }
  auto group_base = [&](const int64_t* st, int key0) -> int64_t {
    if (paged) {
      const int64_t blk = load_invariant_i32(a.block_table, b * a.bt_stride[0] + (int64_t)(key0 >> lp) * a.bt_stride[1]);
      return blk * st[0] + (int64_t)(key0 & ((1 << lp) - 1)) * st[1] + (int64_t)kh * st[2];
    }
    return ((int64_t)r.k_base + key0) * st[1] + (int64_t)kh * st[2];
  };

  // K/V tiles are read with buffer loads.  Each 16-key group gets a scalar
  // resource descriptor whose base is the group's first row and whose size
  // ends with the last valid key of the request, so rows past the keys read
  // as zero in hardware; lane offsets are loop-invariant registers.
  u32x4 kreg[KCH];
  u32x4 vreg[VPT][4];
  uint32_t vmask = ~0u;
  const int64_t safe_v = UNIFORM ? 0 : group_base(a.v_stride, 0);
  // Packed K/V: running address of each group's first key for the current
  // tile, advanced by one tile per load (no per-tile 64-bit products).
  const uint16_t* kcur[KCH];
  const uint16_t* vcur[VPT];
#pragma unroll
  for (int c = 0; c < KCH; ++c) kcur[c] = kg + ((int64_t)r.k_base + kgrp[c]) * a.k_stride[1] + (int64_t)kh * a.k_stride[2];
#pragma unroll
  for (int u = 0; u < VPT; ++u) vcur[u] = vg + ((int64_t)r.k_base + vgrp[u]) * a.v_stride[1] + (int64_t)kh * a.v_stride[2];
  const int64_t kstep = (int64_t)BN * a.k_stride[1], vstep = (int64_t)BN * a.v_stride[1];
  auto group_rsrc = [&](const uint16_t* base, const uint16_t* packed_ptr, const int64_t* st, int key0, int row_elems) {
    const int nvalid = min(max(r.k_len - key0, 0), 16);
    const uint16_t* gptr = paged ? (nvalid > 0 ? base + group_base(st, key0) : base) : packed_ptr;
    const int bytes = nvalid > 0 ? 2 * ((nvalid - 1) * (int)st[1] + row_elems) : 0;
    return __builtin_amdgcn_make_buffer_rsrc((void*)gptr, (short)0, bytes, 0x00020000);
  };
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const auto rsrc = group_rsrc(kg, kcur[c], a.k_stride, t0 + kgrp[c], D);
      kcur[c] += kstep;
      kreg[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, koff[c], 0, 0));
    }
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      if (UNIFORM) {
        const auto rsrc = group_rsrc(vg, vcur[u], a.v_stride, t0 + vgrp[u], D);
        vcur[u] += vstep;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          vreg[u][rr] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff[u][rr], 0, 0));
      } else {
        // D = 64: a wave's V rows span two 16-key groups; per-lane addresses.
        const int uid = 64 * wave_u + PF_THREADS * u + lane;
        const int kgp = uid / (D / 8), dc = uid % (D / 8);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int key = t0 + 4 * kgp + rr;
          const bool ok = vunit[u] && key < r.k_len;
          vreg[u][rr] = *(const u32x4*)(vg + (ok ? row_offset(a.v_stride, key) : safe_v) + dc * 8);
          vmask = ok ? (vmask | (1u << (4 * u + rr))) : (vmask & ~(1u << (4 * u + rr)));
        }
      }
    }
  };
  auto store_tile = [&](int buf) {
    const u32x4 zero = {0u, 0u, 0u, 0u};
    uint16_t* kl = smem + buf * (KTILE + VTILE);
#pragma unroll
    for (int c = 0; c < KCH; ++c) *(u32x4*)(kl + kst[c]) = kreg[c];
    uint16_t* vl = kl + KTILE;
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      if (!vunit[u]) continue;
      if (!UNIFORM) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          if (!((vmask >> (4 * u + rr)) & 1)) vreg[u][rr] = zero;
      }
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t w0 = vreg[u][0][p], w1 = vreg[u][1][p], w2 = vreg[u][2][p], w3 = vreg[u][3][p];
        uint2 even, odd;
        even.x = (w0 & 0xffffu) | (w1 << 16);
        even.y = (w2 & 0xffffu) | (w3 << 16);
        odd.x = (w0 >> 16) | (w1 & 0xffff0000u);
        odd.y = (w2 >> 16) | (w3 & 0xffff0000u);
        *(uint2*)(vl + vst[u] + (2 * p) * VLD) = even;
        *(uint2*)(vl + vst[u] + (2 * p + 1) * VLD) = odd;
      }
    }
  };
  (void)KROWS_W;

  const bool cap = a.softcap > 0.0f;
  const float c_scale = a.softmax_scale * LOG2E;          // raw dot -> log2 units
  const float cap_in = cap ? a.softmax_scale / a.softcap : 0.0f;
  const float cap_out = a.softcap * LOG2E;

  float m_run[NB], l_run[NB];
  f32x16 o[DB][NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    m_run[nb] = -INFINITY;
    l_run[nb] = 0.0f;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[db][nb][i] = 0.0f;
  }

  const bool wave_rows = wq0 < r.q_len;
  const int wave_qabs_lo = wq0 + off;
  const int wave_qabs_hi = min(wq0 + NB * 32, r.q_len) - 1 + off;

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int j = 0; j < n_tiles; ++j) {
    const int buf = j & 1;
    const int t0 = j * BN;
    if (j + 1 < n_tiles) load_tile(t0 + BN);
    const bool active = wave_rows && (!CAUSAL || t0 <= wave_qabs_hi);
    if (active) {
      const uint16_t* kl = smem + buf * (KTILE + VTILE);
      const uint16_t* vl = kl + KTILE;
      f32x16 s[KT][NB];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int i = 0; i < 16; ++i) s[kt][nb][i] = 0.0f;
      const uint16_t* krow = kl + l32 * KLD + 8 * hh;
#pragma unroll
      for (int kk = 0; kk < KST; ++kk)
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          const u32x4 av = *(const u32x4*)(krow + 32 * kt * KLD + 16 * kk);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) s[kt][nb] = mfma32<T>(av, qop[nb][kk], s[kt][nb]);
        }
      const bool need_mask = (t0 + BN > r.k_len) || (CAUSAL && t0 + BN - 1 > wave_qabs_lo);
      u32x4 pop[KT][2][NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (cap) {
#pragma unroll
          for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const float x = s[kt][nb][i] * cap_in;
              const float e = fast_exp2(2.0f * LOG2E * x);
              s[kt][nb][i] = cap_out * (1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f));
            }
        }
        if (need_mask) {
          const int qabs = wq0 + nb * 32 + l32 + off;
#pragma unroll
          for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int key = t0 + 32 * kt + 16 * (i >> 3) + 8 * hh + (i & 7);
              const bool ok = key < r.k_len && (!CAUSAL || key <= qabs);
              if (!ok) s[kt][nb][i] = -INFINITY;
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kt][nb][i]);
        mx = fmaxf(mx, shfl_xor_f(mx, 32));
        const float cand = cap ? mx : mx * c_scale;
        const bool need = cand > m_run[nb] + PF_RESCALE;
        if (__any(need)) {
          const float f = need ? fast_exp2(m_run[nb] - cand) : 1.0f;
          if (need) m_run[nb] = cand;
          l_run[nb] *= f;
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][nb][i] *= f;
        }
        const float mref = m_run[nb] == -INFINITY ? 0.0f : m_run[nb];
        const float sc = cap ? 1.0f : c_scale;
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float p = fast_exp2(fmaf(s[kt][nb][i], sc, -mref));
            s[kt][nb][i] = p;
            psum += p;
          }
        l_run[nb] += psum;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            u32x4 w;
#pragma unroll
            for (int q = 0; q < 4; ++q) w[q] = pack2<T>(s[kt][nb][8 * c + 2 * q], s[kt][nb][8 * c + 2 * q + 1]);
            pop[kt][c][nb] = w;
          }
      }
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const int dim = 32 * db + l32;
            const int chunk = (4 * kt + 2 * c + hh) ^ ((dim >> 4) & 7);
            const u32x4 av = *(const u32x4*)(vl + dim * VLD + 8 * chunk);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) o[db][nb] = mfma32<T>(av, pop[kt][c][nb], o[db][nb]);
          }
    }
    if (j + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: O = O^T / l, LSE = m * ln2 + ln(l).
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const float lt = l_run[nb] + shfl_xor_f(l_run[nb], 32);
    const int row = wq0 + nb * 32 + l32;
    if (row < r.q_len) {
      const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
      const int64_t tq = (int64_t)r.q_begin + row;
      uint16_t* op = (uint16_t*)a.out + tq * a.out_stride[0] + (int64_t)h * a.out_stride[1] + 4 * hh;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint2 w;
          w.x = pack2<T>(o[db][nb][4 * g] * inv, o[db][nb][4 * g + 1] * inv);
          w.y = pack2<T>(o[db][nb][4 * g + 2] * inv, o[db][nb][4 * g + 3] * inv);
          *(uint2*)(op + 32 * db + 8 * g) = w;
        }
      if (hh == 0)
        a.lse[(int64_t)h * a.lse_stride[0] + tq * a.lse_stride[1]] =
            lt > 0.0f ? m_run[nb] * LN2 + logf(lt) : -INFINITY;
    }
  }
}

template <int D> constexpr int nb_for() { return D <= 128 ? FA_PF_NB : 1; }
template <int D> constexpr int kt_for() { return D <= 128 ? FA_PF_KT : 2; }
template <int D> constexpr int minb_for() { return D <= 128 ? FA_PF_MINB : 1; }

template <int D>
constexpr size_t lds_bytes() {
  return 2 * (size_t)(32 * kt_for<D>() * (D + 8) + D * (32 * kt_for<D>() + 8)) * sizeof(uint16_t);
}

using PrefillKernel = void (*)(fa_attn_args, PrefillShape);

template <typename T, int D>
PrefillKernel pick(bool causal) {
  constexpr int NB = nb_for<D>(), KT = kt_for<D>(), MB = minb_for<D>();
  return causal ? prefill_kernel<T, D, NB, KT, MB, true> : prefill_kernel<T, D, NB, KT, MB, false>;
}

PrefillKernel select_prefill(const fa_attn_args& a, int* bm, size_t* lds) {
  const int64_t d = a.head_dim_qk;
  const bool bf = a.q_dtype == FA_BF16;
  const bool causal = a.causal != 0;
  switch (d) {
    case 64: *bm = 128 * nb_for<64>(); *lds = lds_bytes<64>(); return bf ? pick<BF16T, 64>(causal) : pick<F16T, 64>(causal);
    case 128: *bm = 128 * nb_for<128>(); *lds = lds_bytes<128>(); return bf ? pick<BF16T, 128>(causal) : pick<F16T, 128>(causal);
    case 256: *bm = 128 * nb_for<256>(); *lds = lds_bytes<256>(); return bf ? pick<BF16T, 256>(causal) : pick<F16T, 256>(causal);
    default: return nullptr;
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool prefill_ok(const fa_attn_args& a) {
  if (!(a.q_dtype == a.k_dtype && a.k_dtype == a.v_dtype && a.v_dtype == a.out_dtype)) return false;
  if (a.q_dtype != FA_BF16 && a.q_dtype != FA_F16) return false;
  if (a.head_dim_qk != a.head_dim_v) return false;
  if (a.head_dim_qk != 64 && a.head_dim_qk != 128 && a.head_dim_qk != 256) return false;
  if (a.leftpad_k || a.alibi || a.sinks || a.q_descale || a.k_descale || a.v_descale) return false;
  if (a.mask_kind != 0 || a.causal_by_batch || a.window_left != -1 || a.window_right != -1) return false;
  if (a.num_splits != 1) return false;
  if (a.q_stride[2] != 1 || a.k_stride[3] != 1 || a.v_stride[3] != 1 || a.out_stride[2] != 1) return false;
  if (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.v) || ((uintptr_t)a.out & 7u)) return false;
  for (int i = 0; i < 2; ++i)
    if ((a.q_stride[i] * 2) % 16 || (a.out_stride[i] * 2) % 8) return false;
  for (int i = a.page_size ? 0 : 1; i < 3; ++i)
    if ((a.k_stride[i] * 2) % 16 || (a.v_stride[i] * 2) % 16) return false;
  if (a.page_size) {
    if (a.page_size < 16 || (a.page_size & (a.page_size - 1))) return false;
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
  int bm = 0;
  size_t lds = 0;
  const PrefillKernel kern = select_prefill(*a, &bm, &lds);
  PrefillShape shp;
  shp.n_qblocks = (int)fa_ceil_div(a->max_seqlen_q, bm);
  shp.log2_page = 0;
  if (a->page_size)
    while ((1ll << shp.log2_page) < a->page_size) ++shp.log2_page;
  const int64_t pairs = a->batch * a->heads_k;
  const int64_t blocks = fa_ceil_div(pairs, 8) * 8 * shp.n_qblocks * (a->heads_q / a->heads_k);
  FA_REQUIRE(blocks <= 0x7fffffffll, "fa_prefill_fwd: grid too large");
  hipError_t err = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (err != hipSuccess) {
    fa_set_error("fa_prefill_fwd: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(err));
    return FA_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(PF_THREADS), lds, (hipStream_t)stream, *a, shp);
  return fa_check_launch("fa_prefill_fwd");
}
