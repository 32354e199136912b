// Shared device helpers for the elastic sparse attention kernels (gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace esa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Elastic pattern arithmetic.
//
// The reference builds its index set with torch CPU float32 ops
// (elastic_sparse_attention.py:482-533); every op rounds on its own, division
// is IEEE true division and torch.round is round-half-to-even.  The functions
// below evaluate exactly that sequence: contraction is switched off so no
// multiply-add is fused, '/' is the correctly rounded float division hipcc
// emits by default, and rintf is v_rndne_f32 (round half to even).
//
//   alpha  = layer_idx / max(num_layers - 1, 1)      (double, :488-489)
//   a      = f32(alpha), c = f32(w * (1 - alpha))    (scalar casts, :496)
//   end    = max(w - 1, i)                           (:483)
//   pd     = c + f32(f32(end + 1) * a)               (:495-496)
//   st     = max(0, rne(f32(end + 1) - pd))          (:497)
//   sp     = f32(end + 1 - st) / f32(w)              (:498-499)
//   o_j    = st + rne(f32(j) * sp), j = 0..w         (:503-506)
//   idx_j  = rne(f32(o_j * (1 - t)) + f32((o_{j+1} - 1) * t)),
//            t = f32(h) / f32(H - 1) or 0 for H == 1 (:510-526)
//   valid  = idx_j <= i                              (:532)
// ---------------------------------------------------------------------------
struct PatternConsts {
  float a;    // f32(alpha)
  float c;    // f32(w * (1 - alpha))
  int w;      // attention_length
  int H;      // query heads the head interpolation runs over
};

struct HeadWeights {
  float t;    // f32(h) / f32(H - 1)
  float omt;  // f32(1 - t)
};

__device__ __forceinline__ HeadWeights head_weights(const PatternConsts& pc, int h) {
#pragma clang fp contract(off)
  HeadWeights hw;
  if (pc.H > 1) {
    hw.t = (float)h / (float)(pc.H - 1);
    hw.omt = 1.0f - hw.t;
  } else {
    hw.t = 0.0f;
    hw.omt = 1.0f;
  }
  return hw;
}

struct RowParams {
  int st;    // window start
  float sp;  // spacing
};

__device__ __forceinline__ RowParams row_params(const PatternConsts& pc, int i) {
#pragma clang fp contract(off)
  RowParams r;
  int end = i > pc.w - 1 ? i : pc.w - 1;
  float e1 = (float)(end + 1);
  float prod = e1 * pc.a;
  float pd = pc.c + prod;
  float x = e1 - pd;
  float st = rintf(x);
  st = st < 0.0f ? 0.0f : st;
  r.st = (int)st;
  r.sp = (float)(end + 1 - r.st) / (float)pc.w;
  return r;
}

// o_j = st + rne(f32(j) * sp)
__device__ __forceinline__ int oversized(const RowParams& rp, int j) {
#pragma clang fp contract(off)
  float x = (float)j * rp.sp;
  return rp.st + (int)rintf(x);
}

// idx_j from o_j and o_{j+1}
__device__ __forceinline__ int interp_index(int oj, int oj1, const HeadWeights& hw) {
#pragma clang fp contract(off)
  float b = (float)oj * hw.omt;
  float s = (float)(oj1 - 1) * hw.t;
  float f = b + s;
  return (int)rintf(f);
}

// ---------------------------------------------------------------------------
// Small helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(((uint32_t)v) << 16);
}

// Round-to-nearest-even float -> bf16 bits (inputs are finite or inf here).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace esa
