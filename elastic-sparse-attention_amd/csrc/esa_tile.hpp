// Device helpers shared by the block-sparse MFMA kernels (gfx950): LDS chunk
// swizzles, MFMA and packing wrappers, wave reductions, direct HBM -> LDS
// loads, and the walk of one query row's elastic index list through the
// layout's tiles.
#pragma once
#include "esa_internal.hpp"
#include "esa_mma.hpp"

namespace esa {

// Chunk swizzles (chunk index XOR f(row)); both depend only on row bits the
// kernel's row offsets (multiples of 8 for V, 32 for K) leave unchanged.
template <int D>
__device__ __forceinline__ int swz_k(int row) {
  return D == 128 ? (((row & 3) << 2) ^ ((row >> 2) & 3))
                  : ((((row >> 1) & 1) << 2) ^ ((row >> 2) & 3));
}
template <int D>
__device__ __forceinline__ int swz_v(int row) {
  return D == 128 ? ((row & 3) << 2) : (((row >> 1) & 1) << 2);
}

// Rows whose index list is a contiguous run and whose indices are exact in
// float32 (the interpolation of equal integers x reproduces x when x < 2^21).
constexpr int kContigLimit = 1 << 21;
// Lazy rescale threshold (log2 units): the running max moves only when a
// block raises a row's max by more than this, so probabilities stay <= 2^8.
constexpr float kRescaleSlack = 8.0f;
// s_waitcnt with vmcnt(0) and the other counters left alone (gfx9 encoding)
constexpr int kWaitVmcnt0 = 0x0F70;

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// c + lo + hi of a packed bf16 pair, in float32 (v_dot2 with (1, 1))
__device__ __forceinline__ float dot2_bf16(uint32_t pair, float c) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), one, c, false);
}

// max of two floats, neither a signalling NaN, as one v_max_f32: fmaxf of a
// lane swap's results would first quiet each input (a v_max_f32 of the value
// with itself, since the compiler cannot tell they are not signalling NaNs),
// two extra instructions on each reduction's dependent chain.  Scores and
// running maxima are never signalling NaNs, so the result is fmaxf's.
__device__ __forceinline__ float max_nq(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// max of v over lanes l and l ^ 32 (v_permlane32_swap)
__device__ __forceinline__ float half_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return max_nq(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Bits [a - 32 w, b - 32 w] of word w of a 128-bit mask (a <= b, both in [0, 127]).
__device__ __forceinline__ uint32_t range_word(int a, int b, int w) {
  const int lo = max(a - 32 * w, 0);
  const int hi = min(b - 32 * w, 31);
  const int n = hi - lo;
  const uint32_t bits = (0xffffffffu >> ((31 - n) & 31)) << (lo & 31);
  return n >= 0 ? bits : 0u;
}

// S^T accumulator initial values from a lane's masked-key bits nmk (bit
// 8 (r / 4) + r % 4 for register r): -inf where set, else 0.  One v_bfe_i32
// (0 or -1) and one v_and per register; written as inline asm because the
// compiler turns a one-bit sign extract into a test, compare and select.
template <int R>
__device__ __forceinline__ void mask_init(f32x16& s, uint32_t nmk) {
  if constexpr (R < 16) {
    uint32_t v;
    asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(v) : "v"(nmk), "i"(8 * (R / 4) + R % 4));
    s[R] = __uint_as_float(v & 0xff800000u);
    mask_init<R + 1>(s, nmk);
  }
}

// Per-register select masks from a lane's valid-key bits mk (bit
// 8 (r / 4) + r % 4 for register r): -1 for a valid key, 0 for a masked one,
// one v_bfe_i32 each (inline asm on mk only, which is no MFMA result).
template <int R>
__device__ __forceinline__ void key_masks(uint32_t (&m)[16], uint32_t mk) {
  if constexpr (R < 16) {
    asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(m[R]) : "v"(mk), "i"(8 * (R / 4) + R % 4));
    key_masks<R + 1>(m, mk);
  }
}

// Scores of masked keys to -inf after the MFMA: one v_bfi_b32 per register
// (written in C, not asm, so the compiler keeps the wait states between the
// MFMA that writes s and this VALU read of it).  A select rather than an
// additive mask, so a non-finite key row never reaches the score of a row
// that does not list it (-inf + Inf would be NaN).
__device__ __forceinline__ void mask_select(f32x16& s, const uint32_t (&m)[16]) {
#pragma unroll
  for (int r = 0; r < 16; ++r)
    s[r] = __uint_as_float((m[r] & __float_as_uint(s[r])) | (~m[r] & 0xff800000u));
}

__device__ __forceinline__ bool wave_any(bool p) {
  return __builtin_amdgcn_ballot_w64(p) != 0;
}

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(4))) int32_t* cptr_i32;

// 16 bytes per lane from a buffer resource at voffset + soffset straight into
// LDS at dst + 16 * lane (dst uniform)
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t rsrc, uint16_t* dst, int voffset,
                                           int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)dst, 16, voffset, soffset, 0, 0);
}

// One query row's elastic index list, walked through the layout's tiles in
// ascending key order: for each tile, the 128-bit mask of the row's valid keys
// in [k0, k0 + 128).  Rows whose list is a contiguous run (the sliding window
// of layer 0, and the first w - 1 rows of every layer) set a bit range; the
// others carry one pending entry across tiles, so every index is evaluated
// once (the same float32 sequence as the layout builder).
struct RowWalker {
  static constexpr int kNone = 0x7fffffff;
  HeadWeights hw;
  RowParams rp;
  int row, w;
  bool contig;
  int c_lo, c_hi;              // contiguous run [c_lo, c_hi]
  int jp, o_cur, o_next, pend;  // next unplaced entry jp, its index pend

  __device__ __forceinline__ void init(const PatternConsts& pc, int h, int i, bool row_ok) {
    hw = head_weights(pc, h);
    rp = row_params(pc, i);
    row = i;
    w = pc.w;
    contig = row_ok && rp.sp == 1.0f && i < kContigLimit;
    c_lo = rp.st;
    c_hi = min(rp.st + w - 1, i);
    jp = 0;
    o_cur = rp.st;
    o_next = rp.st;
    pend = kNone;
    if (row_ok && !contig) {
      o_next = oversized(rp, 1);
      pend = interp_index(o_cur, o_next, hw);
      if (pend > i) pend = kNone;
    }
  }

  // Valid keys of this row inside [k0, k0 + 32 NW) as NW mask words; spans
  // must come in ascending, non-overlapping order and include every span
  // holding a valid entry of the row.
  template <int NW>
  __device__ __forceinline__ void span(int k0, uint32_t* mb) {
#pragma unroll
    for (int q = 0; q < NW; ++q) mb[q] = 0u;
    if (contig) {
      const int a = max(c_lo, k0) - k0, e = min(c_hi, k0 + 32 * NW - 1) - k0;
      if (a <= e) {
#pragma unroll
        for (int q = 0; q < NW; ++q) mb[q] = range_word(a, e, q);
      }
    }
    while (pend < k0 + 32 * NW) {
      const int rel = pend - k0;
      const uint32_t bit = 1u << (rel & 31);
      const int wsel = rel >> 5;
#pragma unroll
      for (int q = 0; q < NW; ++q) mb[q] |= wsel == q ? bit : 0u;
      if (++jp == w) {
        pend = kNone;
      } else {
        o_cur = o_next;
        o_next = oversized(rp, jp + 1);
        pend = interp_index(o_cur, o_next, hw);
        if (pend > row) pend = kNone;  // indices rise with j: the rest are masked
      }
    }
  }

  // Valid keys of this row inside the 128-key tile [k0, k0 + 128).
  __device__ __forceinline__ void tile(int k0, uint32_t (&mb)[4]) { span<4>(k0, mb); }

  // Two stages of 32 NW keys at ka and kb (kb > ka, or no second stage):
  // mb[0 .. NW) for ka, mb[NW .. 2 NW) for kb; adjacent stages are walked as
  // one span.
  template <int NW>
  __device__ __forceinline__ void stage_pair(int ka, int kb, bool has_b, uint32_t (&mb)[2 * NW]) {
    if (has_b && kb == ka + 32 * NW) {
      span<2 * NW>(ka, mb);
    } else {
      span<NW>(ka, mb);
      if (has_b) {
        span<NW>(kb, mb + NW);
      } else {
#pragma unroll
        for (int q = NW; q < 2 * NW; ++q) mb[q] = 0u;
      }
    }
  }
};

// Online-softmax attention of 32 query rows (one wave) against 32-key blocks
// staged in LDS: the block-sparse forward's per-wave step.
// Each lane owns row l % 32 of the wave and half hf = l / 32 of each block's
// keys.  Per block:
//   S^T = K Q^T    D/16 x v_mfma_f32_32x32x16 (A = K rows from LDS, B = Q
//                  kept in registers for the whole item)
//   softmax        online, log2 domain; the mask enters as the accumulator's
//                  initial value (0 or -inf); a block holding no valid key for
//                  any row of the wave is skipped whole; the running max is
//                  raised only when a row's block max exceeds it by more than
//                  kRescaleSlack, so probabilities stay below 2^8
//   O^T += V^T P^T D/16 x v_mfma_f32_32x32x16 (A = V^T read with
//                  ds_read_b64_tr_b16 from row-major V in LDS, B = P straight
//                  from the S^T accumulators: a key permutation shared by both
//                  operands leaves the contraction unchanged)
// LDS rows are unpadded with XOR-swizzled 16-byte chunks (swz_k / swz_v).
template <int D, Elem E>
struct Rows32 {
  static constexpr int NS = D / 16;  // k-steps of QK^T
  static constexpr int ND = D / 32;  // 32-wide d blocks of PV
  using M = MmaT<E>;
  using V8 = typename M::v8;

  V8 qop[NS];      // Q as the B operand: 8 consecutive d per lane and k-step
  int kaddr[NS];   // K operand read offsets (elements) within a 32-key block
  int vaddr[ND];   // V^T operand read offsets
  f32x16 oacc[ND];
  float m_run;     // running max, log2 units (the same in both halves)
  float l_run;     // running sum of p over this lane's half of the keys (-> lse)
  float n_run;     // the same sum of p rounded to the input type, as PV sees it (-> O)
  float scale;     // sm_scale * log2(e), > 0
  int hf;

  __device__ __forceinline__ void init(int lane, float scale_log2) {
    hf = lane >> 5;
    const int l32 = lane & 31, g4 = lane >> 4, lam = lane & 15;
    scale = scale_log2;
    // K rows l32 at chunk 2 s + hf; V rows 4 hf + lam / 4 (+ 16 u, + 8) at
    // column 32 d + 16 (g4 & 1) + 4 (lam & 3)
#pragma unroll
    for (int s = 0; s < NS; ++s) kaddr[s] = l32 * D + 8 * ((2 * s + hf) ^ swz_k<D>(l32));
    const int vrow = 4 * hf + (lam >> 2);
#pragma unroll
    for (int d = 0; d < ND; ++d) {
      const int col = 32 * d + 16 * (g4 & 1) + 4 * (lam & 3);
      vaddr[d] = vrow * D + 8 * ((col >> 3) ^ swz_v<D>(vrow)) + (col & 7);
    }
    reset();
  }

  __device__ __forceinline__ void reset() {
    m_run = -INFINITY;
    l_run = 0.f;
    n_run = 0.f;
#pragma unroll
    for (int d = 0; d < ND; ++d) oacc[d] = f32x16{};
  }

  // Q row `row` of 16-bit elements (zeros when !ok)
  __device__ __forceinline__ void load_q(const uint16_t* qrow, bool ok) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (ok) raw = *(const u32x4*)(qrow + 16 * s + 8 * hf);
      qop[s] = __builtin_bit_cast(V8, raw);
    }
  }

  // One 32-key block: keys 32 kbl .. 32 kbl + 31 of the LDS buffers (Kb, Vb),
  // whose valid-key bits for this lane's row are mbits (bit k: key k).
  // SAN: the rerun of an item whose output met a non-finite value: masked
  // scores are selected to -inf after the MFMA (instead of entering as the
  // accumulator's -inf start, where a non-finite K value would make NaN of
  // them); the caller has sanitised the staged V rows.  For finite inputs
  // both give the same bits.
  template <bool SAN>
  __device__ __forceinline__ void block(const uint16_t* Kb, const uint16_t* Vb, int kbl,
                                        uint32_t mbits) {
    // lane half hf holds keys 8*(r/4) + 4*hf + r%4 of the block
    const uint32_t mk = mbits >> (4 * hf);
    // a 32 x 32 block in which no row of the wave has a valid key contributes
    // p = 0 to every row: its reads, MFMAs and softmax are all skipped (O, the
    // running max and the sums are unchanged, bit for bit)
    if (!wave_any(mk != 0u)) return;

    // all K operand reads first, so their LDS latency overlaps
    V8 ka[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) ka[s] = *(const V8*)(Kb + kaddr[s] + 32 * kbl * D);
    f32x16 sacc;
    if constexpr (SAN) {
      sacc = f32x16{};
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < NS; ++s) sacc = M::mfma32(ka[s], qop[s], sacc);
      // (the masks are formed after the MFMAs, one register at a time, so the
      // rerun holds no more registers than the first run)
      __builtin_amdgcn_sched_barrier(0);
      uint32_t kmask[16];
      key_masks<0>(kmask, mk);
      mask_select(sacc, kmask);
    } else {
      // the mask enters as the accumulator's initial value: 0 for a valid
      // key, -inf for a masked one
      mask_init<0>(sacc, ~mk);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < NS; ++s) sacc = M::mfma32(ka[s], qop[s], sacc);
    }
    // the V^T operands of this block, read while the softmax runs
    s16x4 va[ND][4];
#pragma unroll
    for (int d = 0; d < ND; ++d) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint16_t* p1 = Vb + vaddr[d] + (32 * kbl + 16 * u) * D;
        va[d][2 * u] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p1);
        va[d][2 * u + 1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1 + 8 * D));
      }
    }
    __builtin_amdgcn_sched_barrier(0);

    uint32_t pw[8];  // P as packed 16-bit pairs: pw[q] holds regs 2q, 2q+1
    // x = scaled score relative to the running max (log2 units); a masked
    // key stays -inf (scale > 0)
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float smax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = __builtin_fmaf(sacc[r], scale, -m_use);
      smax = fmaxf(smax, sacc[r]);
    }
    smax = half_max(smax);
    // raise the running max of a row when this block exceeds it by more
    // than the slack (or when the row sees its first valid key: then the
    // threshold is -inf, and smax > -inf is smax != -inf)
    const float thr = m_run == -INFINITY ? -INFINITY : kRescaleSlack;
    const bool grow = smax > thr;
    if (wave_any(grow)) {
      const float delta = grow ? smax : 0.f;
      // rows that do not grow keep alpha = 1 (m_run may still be -inf there)
      const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - (m_use + delta)) : 1.0f;
      l_run *= alpha;
      n_run *= alpha;
#pragma unroll
      for (int d = 0; d < ND; ++d) oacc[d] *= alpha;
      m_run = grow ? m_use + delta : m_run;
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] -= delta;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float p0 = __builtin_amdgcn_exp2f(sacc[2 * q]);
      const float p1 = __builtin_amdgcn_exp2f(sacc[2 * q + 1]);
      l_run += p0;
      l_run += p1;
      pw[q] = M::pack2(p0, p1);
      // normalise O by the probabilities PV actually used, so a row led by
      // one key reproduces that key's value row
      n_run = M::dot2(pw[q], n_run);
    }

#pragma unroll
    for (int d = 0; d < ND; ++d) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const s16x4 vv[2] = {va[d][2 * u], va[d][2 * u + 1]};
        const V8 a = __builtin_bit_cast(V8, vv);
        const u32x4 pq = {pw[4 * u], pw[4 * u + 1], pw[4 * u + 2], pw[4 * u + 3]};
        oacc[d] = M::mfma32(a, __builtin_bit_cast(V8, pq), oacc[d]);
      }
    }
  }

  // Epilogue: O normalised by the rounded probabilities PV used (a row led by
  // one key reproduces that key's value row), lse by the exact float32 sum
  // (natural log); rows with no valid key get O = 0 and lse = -inf.
  __device__ __forceinline__ void store(uint16_t* orow, float* lse, bool row_ok) {
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float n_tot = n_run + __shfl_xor(n_run, 32, 64);
    if (!row_ok) return;
    const float inv = n_tot > 0.f ? 1.f / n_tot : 0.f;
#pragma unroll
    for (int d = 0; d < ND; ++d) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        typename M::v4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = (typename M::s)(oacc[d][4 * q4 + e] * inv);
        *(typename M::v4*)(orow + 32 * d + 8 * q4 + 4 * hf) = ov;
      }
    }
    if (lse && hf == 0)
      *lse = l_tot > 0.f ? (m_run + __log2f(l_tot)) * 0.69314718055994530942f : -INFINITY;
  }

  // After a rerun with sanitised V: the dims of this lane's output where row
  // i's own entries bring an Inf or NaN of V take the reference's value.
  // vrows: element 0 of key 0 of the (batch, kv head).
  __device__ __forceinline__ void put_nonfinite(uint16_t* orow, const PatternConsts& pc, int h,
                                                int i, const uint16_t* vrows, int64_t vss) {
    int dim0[4 * ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) dim0[4 * d + g] = 32 * d + 8 * g + 4 * hf;
    uint64_t pos, neg, nan;
    nonfinite_v<E>(pc, h, i, vrows, vss, dim0, pos, neg, nan);
    for (uint64_t any = pos | neg | nan; any != 0ull; any &= any - 1ull) {
      const int bit = __builtin_ctzll(any);
      orow[dim0[bit >> 2] + (bit & 3)] = nonfinite_value<E>(pos, neg, nan, bit);
    }
  }
};

}  // namespace esa
