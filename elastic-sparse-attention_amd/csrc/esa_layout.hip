// Elastic index set and block layout builders (gfx950).
//
// indices_kernel   <- _create_elastic_sparse_indices (elastic_sparse_attention.py:470-535)
// tile_bits_kernel, scan_kernel, emit_kernel
//                  -> CSR of active key tiles per (head, query block), derived
//                     from the same index set; no reference counterpart.
#include "esa_internal.hpp"

namespace esa {

// One thread per (h, row, j) entry; consecutive threads write consecutive j,
// so the int32/int64 stores are coalesced.
template <typename IdxT>
__global__ __launch_bounds__(256) void indices_kernel(PatternConsts pc, int row0, int nrows,
                                                      IdxT* __restrict__ indices,
                                                      IdxT* __restrict__ mask) {
  const int h = blockIdx.y;
  const int64_t per_head = (int64_t)nrows * pc.w;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= per_head) return;
  const int r = (int)(e / pc.w);
  const int j = (int)(e - (int64_t)r * pc.w);
  const int i = row0 + r;
  const HeadWeights hw = head_weights(pc, h);
  const RowParams rp = row_params(pc, i);
  const int idx = interp_index(oversized(rp, j), oversized(rp, j + 1), hw);
  const bool valid = idx <= i;
  const int64_t off = (int64_t)h * per_head + e;
  if (indices) indices[off] = (IdxT)(valid ? idx : 0);
  if (mask) mask[off] = (IdxT)(valid ? 1 : 0);
}

// One workgroup per (row, head) of the dense mask <- _create_full_sparse_mask
// (elastic_sparse_attention.py:537-572): the row's ncols bytes are cleared
// (16 bytes per store where the row allows), then every valid entry sets
// the byte of its index, clamped to [0, ncols - 1] as :556 clamps it.  The
// barrier orders the clearing stores before the setting ones.
__global__ __launch_bounds__(256) void dense_mask_kernel(PatternConsts pc, int row0, int ncols,
                                                         uint8_t* __restrict__ mask,
                                                         int64_t stride_h, int64_t stride_s) {
  const int r = blockIdx.x, h = blockIdx.y;
  const int i = row0 + r;
  uint8_t* row = mask + (int64_t)h * stride_h + (int64_t)r * stride_s;
  if (((uintptr_t)row & 15) == 0 && (ncols & 15) == 0) {
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int c = 16 * threadIdx.x; c < ncols; c += 16 * blockDim.x) *(u32x4*)(row + c) = z;
  } else {
    for (int c = threadIdx.x; c < ncols; c += blockDim.x) row[c] = 0;
  }
  __syncthreads();
  const HeadWeights hw = head_weights(pc, h);
  const RowParams rp = row_params(pc, i);
  for (int j = threadIdx.x; j < pc.w; j += blockDim.x) {
    const int idx = interp_index(oversized(rp, j), oversized(rp, j + 1), hw);
    if (idx <= i) row[min(max(idx, 0), ncols - 1)] = 1;
  }
}

// One workgroup per (query block, head): marks the key tiles the block's
// valid entries fall in, in an LDS bitmap, then stores the bitmap and its
// population count.
__global__ __launch_bounds__(256) void tile_bits_kernel(PatternConsts pc, int seq_len, int bm,
                                                        int bn, int nqb, int nwords,
                                                        uint32_t* __restrict__ bits,
                                                        int32_t* __restrict__ counts) {
  extern __shared__ uint32_t sbits[];
  const int qb = blockIdx.x, h = blockIdx.y;
  for (int wd = threadIdx.x; wd < nwords; wd += blockDim.x) sbits[wd] = 0u;
  __syncthreads();
  const HeadWeights hw = head_weights(pc, h);
  const int rows = min(bm, seq_len - qb * bm);
  const int entries = rows * pc.w;
  for (int e = threadIdx.x; e < entries; e += blockDim.x) {
    const int r = e / pc.w, j = e - r * pc.w;
    const int i = qb * bm + r;
    const RowParams rp = row_params(pc, i);
    const int idx = interp_index(oversized(rp, j), oversized(rp, j + 1), hw);
    if (idx <= i) {
      const int kb = idx / bn;  // idx >= 0 for valid entries
      atomicOr(&sbits[kb >> 5], 1u << (kb & 31));
    }
  }
  __syncthreads();
  const int64_t row = (int64_t)h * nqb + qb;
  int cnt = 0;
  for (int wd = threadIdx.x; wd < nwords; wd += blockDim.x) {
    const uint32_t v = sbits[wd];
    bits[row * nwords + wd] = v;
    cnt += __popc(v);
  }
  // block reduction of cnt
  __shared__ int red[256];
  red[threadIdx.x] = cnt;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) counts[row] = red[0];
}

// Single workgroup exclusive scan: row_ptr[0] = 0, row_ptr[k+1] = sum counts[0..k].
__global__ __launch_bounds__(1024) void scan_kernel(const int32_t* __restrict__ counts, int64_t n,
                                                    int32_t* __restrict__ row_ptr) {
  __shared__ int64_t part[1024];
  const int t = threadIdx.x;
  const int64_t chunk = (n + 1023) / 1024;
  const int64_t b0 = min(n, (int64_t)t * chunk), b1 = min(n, b0 + chunk);
  int64_t s = 0;
  for (int64_t k = b0; k < b1; ++k) s += counts[k];
  part[t] = s;
  __syncthreads();
  // Hillis-Steele inclusive scan over 1024 partials
  for (int off = 1; off < 1024; off <<= 1) {
    int64_t v = t >= off ? part[t - off] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  int64_t run = t > 0 ? part[t - 1] : 0;
  if (t == 0) row_ptr[0] = 0;
  for (int64_t k = b0; k < b1; ++k) {
    run += counts[k];
    row_ptr[k + 1] = (int32_t)run;
  }
}

// One workgroup per (query block, head): writes the set bits of the row's
// bitmap, ascending, to col_idx[row_ptr[row] ...].
__global__ __launch_bounds__(256) void emit_kernel(const uint32_t* __restrict__ bits, int nqb,
                                                   int nwords, const int32_t* __restrict__ row_ptr,
                                                   int32_t* __restrict__ col_idx) {
  const int qb = blockIdx.x, h = blockIdx.y;
  const int64_t row = (int64_t)h * nqb + qb;
  const uint32_t* rb = bits + row * nwords;
  const int t = threadIdx.x;
  const int per = (nwords + 255) / 256;
  const int w0 = min(nwords, t * per), w1 = min(nwords, w0 + per);
  int cnt = 0;
  for (int wd = w0; wd < w1; ++wd) cnt += __popc(rb[wd]);
  __shared__ int pre[256];
  pre[t] = cnt;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    int v = t >= off ? pre[t - off] : 0;
    __syncthreads();
    pre[t] += v;
    __syncthreads();
  }
  int pos = row_ptr[row] + (t > 0 ? pre[t - 1] : 0);
  for (int wd = w0; wd < w1; ++wd) {
    uint32_t v = rb[wd];
    while (v) {
      const int b = __ffs(v) - 1;
      col_idx[pos++] = wd * 32 + b;
      v &= v - 1;
    }
  }
}

hipError_t launch_indices(const PatternConsts& pc, int row0, int nrows, void* indices, void* mask,
                          int elem_bytes, hipStream_t stream) {
  const int64_t per_head = (int64_t)nrows * pc.w;
  dim3 grid((unsigned)((per_head + 255) / 256), (unsigned)pc.H);
  if (elem_bytes == 8)
    indices_kernel<int64_t><<<grid, 256, 0, stream>>>(pc, row0, nrows, (int64_t*)indices,
                                                      (int64_t*)mask);
  else
    indices_kernel<int32_t><<<grid, 256, 0, stream>>>(pc, row0, nrows, (int32_t*)indices,
                                                      (int32_t*)mask);
  return hipGetLastError();
}

hipError_t launch_dense_mask(const PatternConsts& pc, int row0, int nrows, int ncols,
                             uint8_t* mask, int64_t stride_h, int64_t stride_s,
                             hipStream_t stream) {
  dim3 grid((unsigned)nrows, (unsigned)pc.H);
  dense_mask_kernel<<<grid, 256, 0, stream>>>(pc, row0, ncols, mask, stride_h, stride_s);
  return hipGetLastError();
}

hipError_t launch_layout(const PatternConsts& pc, const LayoutDims& ld, int32_t* row_ptr,
                         int32_t* col_idx, void* workspace, hipStream_t stream) {
  uint32_t* bits = (uint32_t*)workspace;
  int32_t* counts = (int32_t*)(bits + (int64_t)pc.H * ld.nqb * ld.nwords);
  dim3 grid((unsigned)ld.nqb, (unsigned)pc.H);
  tile_bits_kernel<<<grid, 256, ld.nwords * sizeof(uint32_t), stream>>>(
      pc, ld.seq_len, ld.bm, ld.bn, ld.nqb, ld.nwords, bits, counts);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  scan_kernel<<<1, 1024, 0, stream>>>(counts, (int64_t)pc.H * ld.nqb, row_ptr);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  emit_kernel<<<grid, 256, 0, stream>>>(bits, ld.nqb, ld.nwords, row_ptr, col_idx);
  return hipGetLastError();
}

}  // namespace esa
