// Rate probes (gfx950): dense bf16 MFMA, HBM read, L2 -> LDS or HBM -> LDS
// through the buffer_load ... lds path the MFMA kernels stage K and V with,
// 256-byte row gathers into LDS (the band kernels' pattern) and from HBM
// into registers (the decode step's), and the band kernels' LDS operand
// reads (bank-conflict rates of each read form).
// Built into libesa_probe.so; declared in include/esa_probe.h.
#include <hip/hip_runtime.h>

#include "esa_probe.h"
#include "esa_band.hpp"

namespace esa {
namespace {

constexpr int kThreads = 256;
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
constexpr int kChunk = 16384;  // bytes one workgroup round moves (256 lanes x 4 x 16 B)
// s_waitcnt with vmcnt(8) and the other counters left alone (gfx9 encoding)
constexpr int kWaitVmcnt8 = 0x0F78;

__global__ __launch_bounds__(kThreads) void mfma_probe_kernel(int iters, uint16_t one, float* sink) {
  bf16x8 a;
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = __builtin_bit_cast(__bf16, one);
  f32x16 c[4] = {f32x16{}, f32x16{}, f32x16{}, f32x16{}};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, a, c[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += c[j][r];
  sink[(int64_t)blockIdx.x * kThreads + threadIdx.x] = s;
}

__global__ __launch_bounds__(kThreads) void l2_lds_probe_kernel(const uint16_t* src, int n_chunks,
                                                                int iters, int chunk_stride,
                                                                uint32_t* sink) {
  __shared__ __attribute__((aligned(1024))) uint16_t buf0[kChunk / 2];
  __shared__ __attribute__((aligned(1024))) uint16_t buf1[kChunk / 2];
  const int t = threadIdx.x, wave = t >> 6;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)src, (short)0, n_chunks * kChunk, 0x00020000);
  for (int i = 0; i < iters; ++i) {
    const int c = (int)(((int64_t)blockIdx.x * chunk_stride + i) % n_chunks);
    uint16_t* dst = (i & 1) ? buf1 : buf0;
#pragma unroll
    for (int j = 0; j < 4; ++j)  // load j: bytes (256 j + t) * 16 of the chunk
      load_lds16(rs, dst + (j * kThreads + wave * 64) * 8, (j * kThreads + t) * 16, c * kChunk);
    // at most the last two rounds in flight: the round that wrote this
    // buffer before has landed
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt8);
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  const uint16_t* last = ((iters - 1) & 1) ? buf1 : buf0;
  const u32x4 w = *(const u32x4*)(last + t * 8);  // load 0 of thread t
  uint32_t s = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) s += (w[e] & 0xffffu) + (w[e] >> 16);
  sink[(int64_t)blockIdx.x * kThreads + t] = s;
}

__global__ __launch_bounds__(kThreads) void hbm_read_probe_kernel(const u32x4* src, int64_t n16,
                                                                  uint32_t* sink) {
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  uint32_t acc = 0;
  int64_t k = gid;
  // four loads in flight per thread
  for (; k + 3 * stride < n16; k += 4 * stride) {
    u32x4 x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = __builtin_nontemporal_load(src + k + u * stride);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc += x[u][0] + x[u][1] + x[u][2] + x[u][3];
  }
  for (; k < n16; k += stride) {
    const u32x4 x = __builtin_nontemporal_load(src + k);
    acc += x[0] + x[1] + x[2] + x[3];
  }
  sink[gid] = acc;
}

__global__ __launch_bounds__(kThreads) void gather_lds_probe_kernel(const uint16_t* src, int src_rows,
                                                                    const int32_t* rows,
                                                                    int n_blocks, int iters,
                                                                    uint32_t* sink) {
  __shared__ __attribute__((aligned(1024))) uint16_t buf0[kChunk / 2];
  __shared__ __attribute__((aligned(1024))) uint16_t buf1[kChunk / 2];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int sub = lane >> 4, part = lane & 15;  // row of a DMA, 16-byte piece of it
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)src, (short)0, src_rows * 256, 0x00020000);
  const cptr_i32 rp = (cptr_i32)rows;  // uniform index reads: scalar loads
  for (int i = 0; i < iters; ++i) {
    // this wave's 16 rows of the round (n_blocks blocks of 64 indices)
    const int blk = (int)(((int64_t)blockIdx.x * iters + i) % n_blocks);
    // the 16 indices in one scalar load (64-byte aligned: rows is, and
    // blk * 64 + wave * 16 is a multiple of 16)
    const i32x16 ix = *(const __attribute__((address_space(4))) i32x16*)(rp + blk * 64 + wave * 16);
    uint16_t* dst = (i & 1) ? buf1 : buf0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r0 = ix[4 * j], r1 = ix[4 * j + 1], r2 = ix[4 * j + 2], r3 = ix[4 * j + 3];
      const bool odd = sub & 1, high = sub & 2;
      const int lo = odd ? r1 : r0, hi = odd ? r3 : r2;
      int r = high ? hi : lo;
      r = r < 0 ? 0 : (r >= src_rows ? src_rows - 1 : r);
      load_lds16(rs, dst + (j * kThreads + wave * 64) * 8, r * 256 + part * 16, 0);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt8);
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  const uint16_t* last = ((iters - 1) & 1) ? buf1 : buf0;
  const u32x4 w = *(const u32x4*)(last + t * 8);  // DMA 0 of thread t
  uint32_t s = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) s += (w[e] & 0xffffu) + (w[e] >> 16);
  sink[(int64_t)blockIdx.x * kThreads + t] = s;
}

__global__ __launch_bounds__(kThreads) void gather_probe_kernel(const u32x4* src, int64_t src_rows,
                                                                const int32_t* rows,
                                                                int64_t n_rows, uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const int sub = lane >> 4, part = lane & 15;  // row of an instruction, 16-byte piece
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t wave_id = gid >> 6, n_waves = (int64_t)gridDim.x * (kThreads / 64);
  uint32_t acc = 0;
  // each round of a wave: 8 instructions x 4 rows
  for (int64_t base = wave_id * 32; base < n_rows; base += n_waves * 32) {
    u32x4 x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t r = base + 4 * u + sub;
      int64_t row = r < n_rows ? rows[r] : 0;
      row = row < 0 ? 0 : (row >= src_rows ? src_rows - 1 : row);
      x[u] = src[row * 16 + part];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (base + 4 * u + sub < n_rows) acc += x[u][0] + x[u][1] + x[u][2] + x[u][3];
  }
  sink[gid] = acc;
}

// The band forward's LDS operand reads at D = 128, from one 16-row slot per
// wave (16 rows x 256 bytes, filled with 16-bit ones), `iters` rounds:
//   0: K operand, ds_read_b128, lane (n, q) row n, chunk kswz(n, 4 s + q),
//      s = 0..3 (the kernels' swizzle)
//   1: V^T operand, ds_read_b64_tr_b16, lane x of group q row 4 q + x / 4,
//      dims 32 (x % 4) + 4 s, s = 0..7, chunks by vswz (the kernels')
//   2: V^T operand over contiguous 16-dim slices, dims 16 s + 4 (x % 4),
//      chunks swizzled by 2 (row % 4), so each 16-lane group reads eight
//      chunks in distinct 16-byte bank groups, both halves of each
//   3: pattern 0 without the swizzle (row n, chunk 4 s + q)
// sink[t] = the sum of every 16-bit word thread t read = 32 iters.
template <int MODE>
__global__ __launch_bounds__(kThreads) void lds_read_probe_kernel(int iters, uint32_t* sink) {
  constexpr int D = 128, ROWB = 2 * D, NS = D / 32, NV = D / 16, CW = D / 4;
  __shared__ __attribute__((aligned(1024))) uint16_t slots[4][16 * D];
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, n = lane & 15, q = lane >> 4;
  uint16_t* const slot = slots[wave];
  for (int i = lane; i < 16 * D / 8; i += 64)
    *(u32x4*)(slot + 8 * i) = u32x4{0x00010001u, 0x00010001u, 0x00010001u, 0x00010001u};
  __syncthreads();
  int adr[NV];
#pragma unroll
  for (int s = 0; s < NV; ++s) {
    const int R = 4 * q + (n >> 2);
    if (MODE == 0) adr[s] = n * ROWB + 16 * kswz<D>(n, 4 * (s % NS) + q);
    if (MODE == 3) adr[s] = n * ROWB + 16 * (4 * (s % NS) + q);
    if (MODE == 1) {
      const int dim0 = CW * (n & 3) + 4 * s;
      adr[s] = R * ROWB + 16 * vswz<D>(R, dim0 >> 3) + 2 * (dim0 & 7);
    }
    if (MODE == 2) {
      const int dim0 = 16 * s + 4 * (n & 3);
      adr[s] = R * ROWB + 16 * ((dim0 >> 3) ^ (2 * (R & 3))) + 2 * (dim0 & 7);
    }
  }
  typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
  typedef __attribute__((address_space(3))) char lds_char;
  uint32_t acc = 0;
  for (int it = 0; it < iters; ++it) {
    if constexpr (MODE == 0 || MODE == 3) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const u32x4 v = *(volatile lds_u32x4*)((lds_char*)slot + adr[s]);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc += (v[e] & 0xffffu) + (v[e] >> 16);
      }
    } else {
#pragma unroll
      for (int s = 0; s < NV; ++s) {
        const s16x4 v =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((lds_char*)slot + adr[s]));
#pragma unroll
        for (int e = 0; e < 4; ++e) acc += (uint32_t)(uint16_t)v[e];
        asm volatile("" ::: "memory");
      }
    }
  }
  sink[(int64_t)blockIdx.x * kThreads + t] = acc;
}

esa_status launched() { return hipGetLastError() == hipSuccess ? ESA_OK : ESA_ERR_HIP; }

}  // namespace
}  // namespace esa

using namespace esa;

extern "C" {

esa_status esa_probe_mfma_bf16(int32_t workgroups, int32_t iters, uint16_t one, float* sink,
                               int64_t sink_elems, void* stream) {
  if (!sink) return ESA_ERR_NULL;
  if (workgroups < 1 || workgroups > (1 << 20) || iters < 1 || iters > 16384) return ESA_ERR_SHAPE;
  if (sink_elems < (int64_t)workgroups * kThreads) return ESA_ERR_CAPACITY;
  mfma_probe_kernel<<<workgroups, kThreads, 0, (hipStream_t)stream>>>(iters, one, sink);
  return launched();
}

esa_status esa_probe_l2_to_lds(const void* src, int64_t region_bytes, int32_t workgroups,
                               int32_t iters, int32_t chunk_stride, uint32_t* sink,
                               int64_t sink_elems, void* stream) {
  if (!src || !sink) return ESA_ERR_NULL;
  if (region_bytes < kChunk || region_bytes % kChunk != 0 || region_bytes >= (int64_t(1) << 31) ||
      workgroups < 1 || workgroups > (1 << 20) || iters < 1 || iters > (1 << 20) ||
      chunk_stride < 0 || chunk_stride > (1 << 20))
    return ESA_ERR_SHAPE;
  if ((uintptr_t)src % 16 != 0) return ESA_ERR_ALIGN;
  if (sink_elems < (int64_t)workgroups * kThreads) return ESA_ERR_CAPACITY;
  l2_lds_probe_kernel<<<workgroups, kThreads, 0, (hipStream_t)stream>>>(
      (const uint16_t*)src, (int)(region_bytes / kChunk), iters, chunk_stride, sink);
  return launched();
}

esa_status esa_probe_hbm_read(const void* src, int64_t bytes, int32_t workgroups, uint32_t* sink,
                              int64_t sink_elems, void* stream) {
  if (!src || !sink) return ESA_ERR_NULL;
  if (bytes < 64 || bytes % 64 != 0 || workgroups < 1 || workgroups > (1 << 20))
    return ESA_ERR_SHAPE;
  if ((uintptr_t)src % 16 != 0) return ESA_ERR_ALIGN;
  if (sink_elems < (int64_t)workgroups * kThreads) return ESA_ERR_CAPACITY;
  hbm_read_probe_kernel<<<workgroups, kThreads, 0, (hipStream_t)stream>>>(
      (const u32x4*)src, bytes / 16, sink);
  return launched();
}

esa_status esa_probe_gather_to_lds(const void* src, int64_t src_rows, const int32_t* rows,
                                   int64_t n_rows, int32_t workgroups, int32_t iters,
                                   uint32_t* sink, int64_t sink_elems, void* stream) {
  if (!src || !rows || !sink) return ESA_ERR_NULL;
  if (src_rows < 1 || src_rows * 256 >= (int64_t(1) << 31) || n_rows < 64 || n_rows % 64 != 0 ||
      n_rows >= (int64_t(1) << 31) || workgroups < 1 || workgroups > (1 << 20) || iters < 1 ||
      iters > (1 << 20))
    return ESA_ERR_SHAPE;
  if ((uintptr_t)src % 16 != 0 || (uintptr_t)rows % 64 != 0) return ESA_ERR_ALIGN;
  if (sink_elems < (int64_t)workgroups * kThreads) return ESA_ERR_CAPACITY;
  gather_lds_probe_kernel<<<workgroups, kThreads, 0, (hipStream_t)stream>>>(
      (const uint16_t*)src, (int)src_rows, rows, (int)(n_rows / 64), iters, sink);
  return launched();
}

esa_status esa_probe_gather_read(const void* src, int64_t src_rows, const int32_t* rows,
                                 int64_t n_rows, int32_t workgroups, uint32_t* sink,
                                 int64_t sink_elems, void* stream) {
  if (!src || !rows || !sink) return ESA_ERR_NULL;
  if (src_rows < 1 || n_rows < 1 || workgroups < 1 || workgroups > (1 << 20))
    return ESA_ERR_SHAPE;
  if ((uintptr_t)src % 16 != 0 || (uintptr_t)rows % 4 != 0) return ESA_ERR_ALIGN;
  if (sink_elems < (int64_t)workgroups * kThreads) return ESA_ERR_CAPACITY;
  gather_probe_kernel<<<workgroups, kThreads, 0, (hipStream_t)stream>>>(
      (const u32x4*)src, src_rows, rows, n_rows, sink);
  return launched();
}

esa_status esa_probe_lds_read(int32_t pattern, int32_t workgroups, int32_t iters, uint32_t* sink,
                              int64_t sink_elems, void* stream) {
  using namespace esa;
  if (!sink) return ESA_ERR_NULL;
  if (pattern < 0 || pattern > 3 || workgroups < 1 || workgroups > (1 << 20) || iters < 1 ||
      iters > (1 << 20))
    return ESA_ERR_SHAPE;
  if (sink_elems < (int64_t)workgroups * kThreads) return ESA_ERR_CAPACITY;
  const hipStream_t st = (hipStream_t)stream;
  switch (pattern) {
    case 0: lds_read_probe_kernel<0><<<workgroups, kThreads, 0, st>>>(iters, sink); break;
    case 1: lds_read_probe_kernel<1><<<workgroups, kThreads, 0, st>>>(iters, sink); break;
    case 2: lds_read_probe_kernel<2><<<workgroups, kThreads, 0, st>>>(iters, sink); break;
    default: lds_read_probe_kernel<3><<<workgroups, kThreads, 0, st>>>(iters, sink); break;
  }
  return launched();
}

}  // extern "C"
