// MFMA FlashAttention prefill for gfx950 (bf16 / fp16).
//
// Semantics follow the reference's fast path (flash_attn_mps/_attention.py:149-158,
// flash_attn_mps/kernels/attention_fast.metal:103-597) plus the DIFFKV head
// dims and attention sinks of its tiled path (flash_attn_mps/kernels/
// attention.metal:60-181): packed or paged K/V, GQA, lower-right causality,
// optional softcap, a per-head sink logit that joins the softmax
// denominator only, fp32 softmax and natural-log LSE.  Head dims (Dqk, Dv)
// in {(64,64), (128,128), (256,256), (192,128)}.
//
// gfx950 design
// * A workgroup is W waves; each wave owns NB x 32 query rows of one head.
//   K/V tiles of BN = 32*KT keys are staged in LDS, double buffered; the
//   next tile's global loads are issued before the current tile's MFMAs and
//   only waited for when that tile is written to LDS.
// * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16
//   (A = K rows from LDS, B = Q^T held in registers for the whole kernel).  A
//   lane then holds 32 keys of ONE query column, so the row max / row sum of
//   the softmax are in-lane reductions plus one exchange with lane ^ 32.
// * K rows are stored in LDS at row sigma(r) (bits 2 and 3 of r swapped) so
//   that, in the score layout, every lane's 8 consecutive accumulator values
//   are 8 consecutive keys.  Those 8 probabilities, rounded to bf16/fp16, are
//   directly the B operand of O^T += V^T P^T; V is written transposed into LDS
//   (V^T rows = head dims, 16-byte key chunks XOR-swizzled) so its A operand
//   is one 16-byte LDS read.
// * K/V tiles are read with buffer loads: each 16-key group gets a scalar
//   resource descriptor whose base is the group's first row and whose size
//   ends at the request's last key, so rows past the keys read as zero in
//   hardware and lane offsets are loop-invariant registers.
// * exp2 with softmax_scale*log2(e) folded into one FMA; the running max is
//   only moved (and O rescaled) when a tile raises it by more than 2^8, which
//   keeps probabilities <= 256 and skips almost all rescales.
// * Work is ordered per XCD: each XCD runs whole (request, KV head) pairs one
//   after another, query blocks heaviest-first within a pair (the causal
//   triangle makes late blocks the longest), so resident workgroups share K/V
//   in their XCD's L2.
#include "attn_common.h"

namespace {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

constexpr float PF_RESCALE = 8.0f;  // log2 headroom before the running max moves

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

// True when every wave's rows of every V unit stay inside one 16-key group
// (K chunks always do for the supported head dims), so group storage bases
// are wave-uniform.
constexpr bool groups_uniform(int dq, int dv, int threads) {
  const int kcpr = dq / 8, vcpr = dv / 8;
  for (int c = 0; c * threads < 64 * kcpr; ++c)
    for (int w = 0; w * 64 < threads; ++w) {
      const int s = 64 * w + threads * c, e = s + 63;
      if ((s / kcpr) / 16 != (e / kcpr) / 16) return false;
    }
  for (int u = 0; u * threads < 16 * vcpr; ++u)
    for (int w = 0; w * 64 < threads; ++w) {
      const int s = 64 * w + threads * u;
      if (s >= 16 * vcpr) continue;
      const int e = s + 63 < 16 * vcpr - 1 ? s + 63 : 16 * vcpr - 1;
      if ((4 * (s / vcpr)) / 16 != (4 * (e / vcpr) + 3) / 16) return false;
    }
  return true;
}

constexpr bool k_groups_uniform(int dq, int threads) {
  const int kcpr = dq / 8;
  for (int c = 0; c * threads < 64 * kcpr; ++c)
    for (int w = 0; w * 64 < threads; ++w) {
      const int s = 64 * w + threads * c, e = s + 63;
      if ((s / kcpr) / 16 != (e / kcpr) / 16) return false;
    }
  return true;
}

template <typename T, int DQ, int DV, int NB, int KT, int W, int MINB, bool CAUSAL>
__global__ __launch_bounds__(64 * W, MINB) void prefill_kernel(const fa_attn_args a, const PrefillShape shp) {
  constexpr int THREADS = 64 * W;
  constexpr int BM = W * NB * 32;
  constexpr int BN = 32 * KT;
  constexpr int KST = DQ / 16;                 // k-steps of the QK^T MFMA
  constexpr int DB = DV / 32;                  // 32-row blocks of O^T
  constexpr int KLD = DQ + 8;                  // LDS row stride of K (elements)
  constexpr int VLD = BN + 8;                  // LDS row stride of V^T
  constexpr int KTILE = BN * KLD, VTILE = DV * VLD;
  constexpr int KCPR = DQ / 8, VCPR = DV / 8;  // 16-byte chunks per K / V row
  constexpr int KCH = BN * KCPR / THREADS;     // K chunks per thread
  constexpr int VUNITS = (BN / 4) * VCPR;      // (4 keys x 8 dims) V units per tile
  constexpr int VPT = (VUNITS + THREADS - 1) / THREADS;
  constexpr bool UNIFORM_V = groups_uniform(DQ, DV, THREADS);
  static_assert(KCH >= 1 && BN * KCPR % THREADS == 0, "K staging shape");
  static_assert(k_groups_uniform(DQ, THREADS), "K chunks must stay inside 16-key groups");
  static_assert(BN == 64, "the V^T swizzle assumes 8 key chunks per row");

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave_u = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index as a scalar
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
  const int kh = (int)(pair % a.heads_k);
  const int h = kh * G + rem % G;
  const RequestInfo r = load_request(a, b);
  if ((a.flags & FA_FLAG_SKIP_SINGLE_QUERY) && r.q_len == 1) return;   // the decode kernel owns it
  const int q0 = qb * BM;
  if (q0 >= r.q_len) return;
  const int off = r.k_len - r.q_len;   // absolute position of query row i is i + off
  int kv_end = r.k_len;
  if (CAUSAL) kv_end = min(kv_end, min(q0 + BM, r.q_len) - 1 + off + 1);
  const int n_tiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;

  const uint16_t* qg = (const uint16_t*)a.q;
  const uint16_t* kg = (const uint16_t*)a.k;
  const uint16_t* vg = (const uint16_t*)a.v;

  // Q^T operand for the whole kernel: lane holds Q[row][16kk + 8hh .. +8].
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
  // Storage offset (elements) of key `key`; per lane only for V layouts whose
  // wave rows can span two 16-key groups (Dv = 64).
  auto row_offset = [&](const int64_t* st, int key) -> int64_t {
    if (paged) {
      const int page = key >> lp;
      const int64_t blk = a.block_table[b * a.bt_stride[0] + (int64_t)page * a.bt_stride[1]];
      return blk * st[0] + (int64_t)(key - (page << lp)) * st[1] + (int64_t)kh * st[2];
    }
    return ((int64_t)r.k_base + key) * st[1] + (int64_t)kh * st[2];
  };
  auto group_base = [&](const int64_t* st, int key0) -> int64_t {
    if (paged) {
      const int64_t blk = load_invariant_i32(a.block_table, b * a.bt_stride[0] + (int64_t)(key0 >> lp) * a.bt_stride[1]);
      return blk * st[0] + (int64_t)(key0 & ((1 << lp) - 1)) * st[1] + (int64_t)kh * st[2];
    }
    return ((int64_t)r.k_base + key0) * st[1] + (int64_t)kh * st[2];
  };

  // Staging layout.  K: chunk c of a thread is 16 bytes of row idx / KCPR at
  // column 8 * (idx % KCPR), idx = 64 * wave + THREADS * c + lane, stored at
  // LDS row sigma(row).  V: unit u of a thread covers 4 keys x 8 dims with
  // the dims fastest across lanes (coalesced global reads).
  int kgrp[KCH], koff[KCH], kst[KCH];
#pragma unroll
  for (int c = 0; c < KCH; ++c) {
    const int idx0 = 64 * wave_u + THREADS * c;
    const int idx = idx0 + lane;
    const int row = idx / KCPR, col = idx % KCPR;
    kgrp[c] = (idx0 / KCPR) & ~15;
    koff[c] = 2 * ((row - kgrp[c]) * (int)a.k_stride[1] + col * 8);   // bytes
    kst[c] = sigma(row) * KLD + col * 8;
  }
  int vgrp[VPT], voff[VPT][4], vst[VPT];
  bool vunit[VPT];
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const int uid0 = 64 * wave_u + THREADS * u;
    const int uid = uid0 + lane;
    const int kgp = uid / VCPR, dc = uid % VCPR;
    vunit[u] = uid < VUNITS;
    vgrp[u] = (4 * (uid0 / VCPR)) & ~15;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) voff[u][rr] = 2 * ((4 * kgp + rr - vgrp[u]) * (int)a.v_stride[1] + dc * 8);
    // V^T element (dim, key) lives at dim*VLD + 8*((key/8) ^ ((dim/16) & 7)) + key%8.
    vst[u] = 8 * dc * VLD + 8 * ((kgp >> 1) ^ ((dc >> 1) & 7)) + 4 * (kgp & 1);
  }

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

  u32x4 kreg[KCH];
  u32x4 vreg[VPT][4];
  uint32_t vmask = ~0u;
  const int64_t safe_v = UNIFORM_V ? 0 : group_base(a.v_stride, 0);
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const auto rsrc = group_rsrc(kg, kcur[c], a.k_stride, t0 + kgrp[c], DQ);
      kcur[c] += kstep;
      kreg[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, koff[c], 0, 0));
    }
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      if (UNIFORM_V) {
        const auto rsrc = group_rsrc(vg, vcur[u], a.v_stride, t0 + vgrp[u], DV);
        vcur[u] += vstep;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          vreg[u][rr] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff[u][rr], 0, 0));
      } else {
        const int uid = 64 * wave_u + THREADS * u + lane;
        const int kgp = uid / VCPR, dc = uid % VCPR;
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
      if (!UNIFORM_V) {
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

  const bool cap = a.softcap > 0.0f;
  const float c_scale = a.softmax_scale * LOG2E;          // raw dot -> log2 units
  const float cap_in = cap ? a.softmax_scale / a.softcap : 0.0f;
  const float cap_out = a.softcap * LOG2E;
  // A sink logit seeds the running state (max = sink, sum = 1) of every row.
  const float sink2 = a.sinks ? a.sinks[(int64_t)h * a.sink_stride] * LOG2E : -INFINITY;

  float m_run[NB], l_run[NB];
  f32x16 o[DB][NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    m_run[nb] = sink2;
    l_run[nb] = (a.sinks && hh == 0) ? 1.0f : 0.0f;
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

// Tile shape per head-dim pair: NB query blocks per wave, W waves per
// workgroup, MINB workgroups per CU.  Two waves per SIMD either as two
// 4-wave workgroups (when LDS holds two double-buffered tile pairs) or as
// one 8-wave workgroup sharing its tiles.
template <int DQ, int DV> struct PrefillTile;
template <> struct PrefillTile<64, 64> { static constexpr int NB = 1, W = 4, MINB = 2; };
template <> struct PrefillTile<128, 128> { static constexpr int NB = 1, W = 4, MINB = 2; };
template <> struct PrefillTile<192, 128> { static constexpr int NB = 1, W = 8, MINB = 1; };
template <> struct PrefillTile<256, 256> { static constexpr int NB = 1, W = 4, MINB = 1; };

template <int DQ, int DV>
constexpr size_t lds_bytes() {
  return 2 * (size_t)(64 * (DQ + 8) + DV * (64 + 8)) * sizeof(uint16_t);
}

using PrefillKernel = void (*)(fa_attn_args, PrefillShape);

struct PrefillChoice {
  PrefillKernel kern;
  int bm, threads;
  size_t lds;
};

template <typename T, int DQ, int DV>
PrefillChoice pick(bool causal) {
  using S = PrefillTile<DQ, DV>;
  PrefillChoice c;
  c.kern = causal ? prefill_kernel<T, DQ, DV, S::NB, 2, S::W, S::MINB, true>
                  : prefill_kernel<T, DQ, DV, S::NB, 2, S::W, S::MINB, false>;
  c.bm = 32 * S::NB * S::W;
  c.threads = 64 * S::W;
  c.lds = lds_bytes<DQ, DV>();
  return c;
}

template <typename T>
PrefillChoice pick_dims(int64_t dq, int64_t dv, bool causal) {
  if (dq == 64 && dv == 64) return pick<T, 64, 64>(causal);
  if (dq == 128 && dv == 128) return pick<T, 128, 128>(causal);
  if (dq == 192 && dv == 128) return pick<T, 192, 128>(causal);
  if (dq == 256 && dv == 256) return pick<T, 256, 256>(causal);
  return PrefillChoice{nullptr, 0, 0, 0};
}

PrefillChoice select_prefill(const fa_attn_args& a) {
  const bool causal = a.causal != 0;
  return a.q_dtype == FA_BF16 ? pick_dims<BF16T>(a.head_dim_qk, a.head_dim_v, causal)
                              : pick_dims<F16T>(a.head_dim_qk, a.head_dim_v, causal);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool prefill_ok(const fa_attn_args& a) {
  if (!(a.q_dtype == a.k_dtype && a.k_dtype == a.v_dtype && a.v_dtype == a.out_dtype)) return false;
  if (a.q_dtype != FA_BF16 && a.q_dtype != FA_F16) return false;
  const int64_t dq = a.head_dim_qk, dv = a.head_dim_v;
  if (!((dq == dv && (dq == 64 || dq == 128 || dq == 256)) || (dq == 192 && dv == 128))) return false;
  if (a.leftpad_k || a.alibi || a.q_descale || a.k_descale || a.v_descale) return false;
  if (a.mask_kind != 0 || a.causal_by_batch || a.window_left != -1 || a.window_right != -1) return false;
  if (a.num_splits != 1) return false;
  if (a.q_stride[2] != 1 || a.k_stride[3] != 1 || a.v_stride[3] != 1 || a.out_stride[2] != 1) return false;
  if (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.v) || ((uintptr_t)a.out & 7u)) return false;
  for (int i = 0; i < 2; ++i)
    if ((a.q_stride[i] * 2) % 16 || (a.out_stride[i] * 2) % 8) return false;
  for (int i = a.page_size ? 0 : 1; i < 3; ++i)
    if ((a.k_stride[i] * 2) % 16 || (a.v_stride[i] * 2) % 16) return false;
  // Group-bounded buffer loads need non-overlapping rows and 16-row groups
  // that span less than 2 GiB.
  if (a.k_stride[1] < dq || a.v_stride[1] < dv) return false;
  if (16 * a.k_stride[1] * 2 >= 0x7fffffffll || 16 * a.v_stride[1] * 2 >= 0x7fffffffll) return false;
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
  const PrefillChoice ch = select_prefill(*a);
  PrefillShape shp;
  shp.n_qblocks = (int)fa_ceil_div(a->max_seqlen_q, ch.bm);
  shp.log2_page = 0;
  if (a->page_size)
    while ((1ll << shp.log2_page) < a->page_size) ++shp.log2_page;
  const int64_t pairs = a->batch * a->heads_k;
  const int64_t blocks = fa_ceil_div(pairs, 8) * 8 * shp.n_qblocks * (a->heads_q / a->heads_k);
  FA_REQUIRE(blocks <= 0x7fffffffll, "fa_prefill_fwd: grid too large");
  hipError_t err = hipFuncSetAttribute((const void*)ch.kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)ch.lds);
  if (err != hipSuccess) {
    fa_set_error("fa_prefill_fwd: cannot reserve %zu bytes of LDS: %s", ch.lds, hipGetErrorString(err));
    return FA_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(ch.kern, dim3((unsigned)blocks), dim3(ch.threads), ch.lds, (hipStream_t)stream, *a, shp);
  return fa_check_launch("fa_prefill_fwd");
}
