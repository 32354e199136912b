// MFMA operand traits of the 16-bit input types (gfx950): the MFMA kernels
// take bfloat16 or float16 q, k, v and run the same tiles on
// v_mfma_f32_{32x32x16,16x16x32}_{bf16,f16} with float32 accumulation; the
// probabilities (and dS in the backward) enter PV as the input type, rounded
// to nearest even, and outputs are stored in it.
#pragma once
#include "esa_elem.hpp"

namespace esa {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <Elem E>
struct MmaT;

template <>
struct MmaT<Elem::bf16> {
  using v8 = bf16x8;
  using v4 = bf16x4;
  using s = __bf16;
  __device__ static __forceinline__ f32x16 mfma32(const v8& a, const v8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ f32x4 mfma16(const v8& a, const v8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // two floats as a packed pair (lo in the low half)
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    bf16x2 v;
    v[0] = (__bf16)lo;
    v[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
  // c + lo + hi of a packed pair, in float32 (v_dot2 with (1, 1))
  __device__ static __forceinline__ float dot2(uint32_t pair, float c) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), one, c, false);
  }
  __device__ static __forceinline__ uint16_t bits(float f) { return f32_to_bf16_bits(f); }
  __device__ static __forceinline__ float val(uint32_t b16) { return __uint_as_float(b16 << 16); }
  // exponent field of a packed pair, and its lowest bit in each half
  static constexpr uint32_t kExp2 = 0x7F807F80u, kExpLsb2 = 0x00800080u;
  static constexpr uint16_t kPosInf = 0x7F80, kNegInf = 0xFF80, kNaN = 0x7FC0;
};

template <>
struct MmaT<Elem::f16> {
  using v8 = f16x8;
  using v4 = f16x4;
  using s = _Float16;
  __device__ static __forceinline__ f32x16 mfma32(const v8& a, const v8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ f32x4 mfma16(const v8& a, const v8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    f16x2 v;
    v[0] = (_Float16)lo;
    v[1] = (_Float16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static __forceinline__ float dot2(uint32_t pair, float c) {
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pair), one, c, false);
  }
  __device__ static __forceinline__ uint16_t bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
  __device__ static __forceinline__ float val(uint32_t b16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)b16);
  }
  static constexpr uint32_t kExp2 = 0x7C007C00u, kExpLsb2 = 0x04000400u;
  static constexpr uint16_t kPosInf = 0x7C00, kNegInf = 0xFC00, kNaN = 0x7E00;
};

// Non-finite values in the MFMA kernels.  The reference gathers only the
// K / V rows a query row lists (elastic_sparse_attention.py:131-133, :152-154),
// so an Inf or NaN there reaches exactly the rows that list it; a staged key
// block or band also holds rows a query row does not list, which meet p = 0
// in P V, and 0 * Inf is NaN.  The kernels therefore check their output rows
// at the end (a sum of the accumulators is non-finite exactly when one of
// them is, or when the sum overflows) and, only then, run the rows again with
// the staged V operands sanitised and put the reference's non-finite values
// back from the rows' own entries (nonfinite_v below).

// x with every non-finite 16-bit half (exponent all ones) replaced by +0:
// adding the exponent's lowest bit to the exponent field carries into the
// half's top bit exactly when the field is all ones.
template <Elem E>
__device__ __forceinline__ uint32_t sanitize2(uint32_t x) {
  const uint32_t t = (x & MmaT<E>::kExp2) + MmaT<E>::kExpLsb2;
  const uint32_t f = (t >> 15) & 0x00010001u;  // bit 0 / 16: that half is non-finite
  const uint32_t m = (f << 16) - f;             // f * 0xFFFF: the flagged halves' bits
  return x & ~m;
}

// Is some value of v non-finite (or does their sum overflow)?  A balanced sum
// of the accumulators: Inf and NaN survive addition, so a finite sum means
// every value is finite.
template <int N>
__device__ __forceinline__ bool sum_finite(const f32x4 (&v)[N]) {
  f32x4 t[N];
#pragma unroll
  for (int s = 0; s < N; ++s) t[s] = v[s];
#pragma unroll
  for (int w = N / 2; w >= 1; w /= 2)
#pragma unroll
    for (int s = 0; s < w; ++s) t[s] += t[s + w];
  return __builtin_isfinite((t[0][0] + t[0][1]) + (t[0][2] + t[0][3]));
}
template <int N>
__device__ __forceinline__ bool sum_finite(const f32x16 (&v)[N]) {
  f32x16 t[N];
#pragma unroll
  for (int s = 0; s < N; ++s) t[s] = v[s];
#pragma unroll
  for (int w = N / 2; w >= 1; w /= 2)
#pragma unroll
    for (int s = 0; s < w; ++s) t[s] += t[s + w];
  f32x4 u;
#pragma unroll
  for (int e = 0; e < 4; ++e) u[e] = (t[0][e] + t[0][4 + e]) + (t[0][8 + e] + t[0][12 + e]);
  return __builtin_isfinite((u[0] + u[1]) + (u[2] + u[3]));
}

// The non-finite V values query row i of head h lists: for every valid entry
// of its index list (the pattern's recipe, elastic_sparse_attention.py:
// 482-535; prefill rows, so every index lies below kv_len), the four V
// elements at dims dim0[g] .. dim0[g] + 3 of the entry's key row are checked;
// bit 4 g + e of pos / neg / nan is set when some entry brings +Inf / -Inf /
// NaN at dim0[g] + e.  vrows: element 0 of key 0 of the (batch, kv head).
template <Elem E, int NG>
__device__ __forceinline__ void nonfinite_v(const PatternConsts& pc, int h, int i,
                                            const uint16_t* vrows, int64_t vss,
                                            const int (&dim0)[NG], uint64_t& pos,
                                            uint64_t& neg, uint64_t& nan) {
  static_assert(NG <= 16, "64 dims per lane");
  pos = neg = nan = 0ull;
  const HeadWeights hw = head_weights(pc, h);
  const RowParams rp = row_params(pc, i);
  int o_cur = oversized(rp, 0);
  for (int j = 0; j < pc.w; ++j) {
    const int o_nxt = oversized(rp, j + 1);
    const int idx = interp_index(o_cur, o_nxt, hw);
    o_cur = o_nxt;
    if (idx > i) break;  // indices rise with j: the rest are masked
    const uint16_t* vr = vrows + (int64_t)idx * vss;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const u32x2 w = *(const u32x2*)(vr + dim0[g]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t x = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        const uint32_t ex = MmaT<E>::kExp2 & 0xFFFFu;
        if ((x & ex) == ex) {
          const uint64_t bit = 1ull << (4 * g + e);
          if (x & (ex ^ 0x7FFFu)) nan |= bit;   // mantissa bits set
          else if (x & 0x8000u) neg |= bit;
          else pos |= bit;
        }
      }
    }
  }
}

// The reference's value at a dim where the row's entries bring non-finite V
// values (each with p > 0): NaN if one is NaN or both infinities meet, else
// the infinity.  (Where such an entry's probability underflows to 0, the
// reference gets NaN from 0 * Inf; here the infinity stands.)
template <Elem E>
__device__ __forceinline__ uint16_t nonfinite_value(uint64_t pos, uint64_t neg, uint64_t nan,
                                                    int b) {
  const bool p = (pos >> b) & 1, n = (neg >> b) & 1, x = (nan >> b) & 1;
  return (x || (p && n)) ? MmaT<E>::kNaN : (p ? MmaT<E>::kPosInf : MmaT<E>::kNegInf);
}

}  // namespace esa
