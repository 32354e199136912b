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
};

}  // namespace esa
