// Device helpers shared by the block-sparse MFMA kernels (gfx950): LDS chunk
// swizzles, MFMA and packing wrappers, wave reductions, direct HBM -> LDS
// loads, and the walk of one query row's elastic index list through the
// layout's tiles.
#pragma once
#include "esa_internal.hpp"

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

// max of v over lanes l and l ^ 32 (v_permlane32_swap)
__device__ __forceinline__ float half_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
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

}  // namespace esa
