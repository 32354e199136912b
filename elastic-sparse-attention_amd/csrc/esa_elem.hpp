// Element types of q, k, v, o and the gradients: float32, bfloat16 and
// float16, all computed in float32 (the reference's Triton kernel loads any
// float type, accumulates in float32 and stores in the output's dtype,
// elastic_sparse_attention.py:114, :137, :163).  Rounding to a 16-bit type is
// round-to-nearest-even.
#pragma once
#include "esa_common.hpp"

namespace esa {

enum class Elem { f32 = 0, bf16 = 1, f16 = 2 };

template <Elem E>
struct ElemT;

template <>
struct ElemT<Elem::f32> {
  using T = float;
  static constexpr int kBytes = 4;
  static constexpr int kPerChunk = 4;  // elements in 16 bytes
  __device__ static __forceinline__ float load(const T* p) { return *p; }
  __device__ static __forceinline__ void store(T* p, float v) { *p = v; }
  // element e of a 16-byte chunk
  __device__ static __forceinline__ float chunk(const u32x4& raw, int e) {
    return __uint_as_float(raw[e]);
  }
  // 16 bytes from kPerChunk floats
  __device__ static __forceinline__ u32x4 pack_chunk(const float* x) {
    return u32x4{__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                 __float_as_uint(x[3])};
  }
};

template <>
struct ElemT<Elem::bf16> {
  using T = uint16_t;
  static constexpr int kBytes = 2;
  static constexpr int kPerChunk = 8;
  __device__ static __forceinline__ float load(const T* p) { return bf16_to_f32(*p); }
  __device__ static __forceinline__ void store(T* p, float v) { *p = f32_to_bf16_bits(v); }
  __device__ static __forceinline__ float chunk(const u32x4& raw, int e) {
    return __uint_as_float((e & 1) ? (raw[e / 2] & 0xffff0000u) : (raw[e / 2] << 16));
  }
  __device__ static __forceinline__ u32x4 pack_chunk(const float* x) {
    u32x4 w;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      w[q] = (uint32_t)f32_to_bf16_bits(x[2 * q]) | ((uint32_t)f32_to_bf16_bits(x[2 * q + 1]) << 16);
    return w;
  }
};

template <>
struct ElemT<Elem::f16> {
  using T = uint16_t;
  static constexpr int kBytes = 2;
  static constexpr int kPerChunk = 8;
  __device__ static __forceinline__ float h2f(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
  }
  __device__ static __forceinline__ uint16_t f2h(float v) {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  }
  __device__ static __forceinline__ float load(const T* p) { return h2f(*p); }
  __device__ static __forceinline__ void store(T* p, float v) { *p = f2h(v); }
  __device__ static __forceinline__ float chunk(const u32x4& raw, int e) {
    return h2f((e & 1) ? (raw[e / 2] >> 16) : (raw[e / 2] & 0xffffu));
  }
  __device__ static __forceinline__ u32x4 pack_chunk(const float* x) {
    u32x4 w;
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = (uint32_t)f2h(x[2 * q]) | ((uint32_t)f2h(x[2 * q + 1]) << 16);
    return w;
  }
};

// Integer entry of an index or mask array of 1, 4 or 8 bytes per element.
__device__ __forceinline__ int64_t load_int_any(const void* base, int bytes, int64_t i) {
  if (bytes == 8) return ((const int64_t*)base)[i];
  if (bytes == 4) return ((const int32_t*)base)[i];
  return ((const uint8_t*)base)[i];
}

// Counter-based keep decision of attention dropout for entry `idx` of a call
// seeded with `seed`: the SplitMix64 output function (Steele, Lea and Flood,
// "Fast splittable pseudorandom number generators", OOPSLA 2014) of
// seed + (idx + 1) * golden gamma, top 24 bits as a uniform in [0, 1).  The
// forward, the weights and the backward evaluate the same function, so they
// agree on every entry's mask.
__device__ __forceinline__ bool dropout_keep(uint64_t seed, uint64_t idx, float p_drop) {
  uint64_t z = seed + (idx + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  const float u = (float)(uint32_t)(z >> 40) * (1.0f / 16777216.0f);
  return u >= p_drop;
}

}  // namespace esa
