// Receptive-field reachability through the elastic layers (gfx950).
//
// Replaces check_attention_holes_pytorch (check_attn_hole.py:53-180), which
// materialises every layer's [H, L, w] int64 index set on the device (8.6 GB
// for 8 layers at L = 131072, H = 8, w = 64) and grows a boolean set with
// gathers and unique().  Here the set is a bitmap over the history (bit j of
// word j / 32 = token j) and one layer is one pass over it:
//
//   reach_step_kernel  a workgroup owns kTokensPerWg consecutive source
//                      tokens and one window of kWinWords bitmap words.  Each
//                      lane takes one source token at a time; if the token is
//                      in `src`, the lane regenerates its w elastic indices for
//                      every head (the bit-exact float32 sequence the layout
//                      builder uses) and ORs the valid ones that fall in the
//                      window into an LDS copy of the window (ds_or_b32); a
//                      contiguous index run (the sliding window of layer 0, the
//                      dense prefix of rows below w - 1) is ORed as whole-word
//                      masks instead.  The workgroup then ORs its nonzero LDS
//                      words into `dst`, which holds a copy of `src`.
//   popcount_kernel    the set size after the layer
//
// Reading `src` and writing `dst` keeps the reference's layer semantics: the
// sources of a layer are the tokens reached before it, not those it adds.
#include "esa_tile.hpp"

namespace esa {

namespace {

constexpr int kWinWords = 8192;       // 32 KB of LDS: 262144 tokens per window
constexpr int kTokensPerWg = 1024;    // 4 source tokens per lane

__device__ __forceinline__ void or_range(uint32_t* win, int lo_tok, int hi_tok, int wlo_tok) {
  // tokens [lo_tok, hi_tok], already clipped to the window
  const int a = lo_tok - wlo_tok, b = hi_tok - wlo_tok;
  for (int wd = a >> 5; wd <= (b >> 5); ++wd) {
    const int lo = max(a - 32 * wd, 0), hi = min(b - 32 * wd, 31);
    const uint32_t m = (hi == 31 ? 0xffffffffu : ((1u << (hi + 1)) - 1u)) & ~((1u << lo) - 1u);
    atomicOr(&win[wd], m);
  }
}

}  // namespace

__global__ __launch_bounds__(256) void reach_init_kernel(uint32_t* bits, int nwords, int position,
                                                         int32_t* counts, int ncounts) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t < nwords) bits[t] = (t == (position >> 5)) ? (1u << (position & 31)) : 0u;
  if (counts && t < ncounts) counts[t] = 0;
}

__global__ __launch_bounds__(256) void reach_copy_kernel(uint32_t* dst, const uint32_t* src,
                                                         int nwords) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t < nwords) dst[t] = src[t];
}

// n = position + 1 tokens of history; only sources in [src_lo, src_hi) run
// (the last layer's only source is the position itself).
__global__ __launch_bounds__(256) void reach_step_kernel(PatternConsts pc, int n, int src_lo,
                                                         int src_hi, const uint32_t* __restrict__ src,
                                                         uint32_t* __restrict__ dst) {
  __shared__ uint32_t win[kWinWords];
  const int wlo_word = blockIdx.y * kWinWords;
  const int nwords = (n + 31) >> 5;
  const int wwords = min(kWinWords, nwords - wlo_word);
  if (wwords <= 0) return;
  const int wlo_tok = wlo_word * 32;
  const int whi_tok = min(n, (wlo_word + wwords) * 32) - 1;  // last token of the window
  const int t0 = src_lo + blockIdx.x * kTokensPerWg;
  if (t0 >= src_hi) return;
  // a source reaches only tokens <= itself: skip windows past the last source
  if (wlo_tok > min(src_hi, t0 + kTokensPerWg) - 1) return;

  for (int k = threadIdx.x; k < wwords; k += 256) win[k] = 0u;
  __syncthreads();

  for (int s = 0; s < kTokensPerWg / 256; ++s) {
    const int i = t0 + s * 256 + threadIdx.x;
    if (i >= src_hi) break;
    if (!((src[i >> 5] >> (i & 31)) & 1u)) continue;
    const RowParams rp = row_params(pc, i);
    if (rp.sp == 1.0f && i < kContigLimit) {
      // indices st .. st + w - 1 for every head, valid up to i
      const int lo = max(rp.st, wlo_tok), hi = min(min(rp.st + pc.w - 1, i), whi_tok);
      if (lo <= hi) or_range(win, lo, hi, wlo_tok);
      continue;
    }
    if (rp.st > whi_tok) continue;  // every index is >= st
    for (int h = 0; h < pc.H; ++h) {
      const HeadWeights hw = head_weights(pc, h);
      int oj = oversized(rp, 0);
      for (int j = 0; j < pc.w; ++j) {
        const int oj1 = oversized(rp, j + 1);
        const int idx = interp_index(oj, oj1, hw);
        oj = oj1;
        // valid: 0 <= idx <= i (check_attn_hole.py:49); all valid indices < n
        if (idx >= 0 && idx <= i && idx >= wlo_tok && idx <= whi_tok) {
          const int r = idx - wlo_tok;
          atomicOr(&win[r >> 5], 1u << (r & 31));
        }
      }
    }
  }
  __syncthreads();
  for (int k = threadIdx.x; k < wwords; k += 256) {
    const uint32_t v = win[k];
    if (v) atomicOr(&dst[wlo_word + k], v);
  }
}

__global__ __launch_bounds__(256) void reach_popcount_kernel(const uint32_t* bits, int nwords,
                                                             int32_t* count) {
  int c = 0;
  for (int t = blockIdx.x * 256 + threadIdx.x; t < nwords; t += gridDim.x * 256)
    c += __popc(bits[t]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off, 64);
  if ((threadIdx.x & 63) == 0 && c) atomicAdd(count, c);
}

hipError_t launch_reachability(const PatternConsts* layers, int num_layers, int position,
                               uint32_t* reach, uint32_t* work, int32_t* counts,
                               hipStream_t stream) {
  const int n = position + 1;
  const int nwords = (n + 31) >> 5;
  const unsigned wgs_words = (unsigned)((nwords + 255) / 256);
  // every step writes the buffer it did not read; start so that the last
  // step writes `reach`
  uint32_t* cur = (num_layers % 2 == 0) ? reach : work;
  uint32_t* nxt = (num_layers % 2 == 0) ? work : reach;
  reach_init_kernel<<<dim3(std::max(wgs_words, (unsigned)((num_layers + 255) / 256))), 256, 0,
                      stream>>>(cur, nwords, position, counts, counts ? num_layers : 0);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const unsigned nwin = (unsigned)((nwords + kWinWords - 1) / kWinWords);
  for (int k = 0; k < num_layers; ++k) {
    // layers[k] is layer num_layers - 1 - k; the last layer's only source is
    // the position itself (check_attn_hole.py:106-114)
    const int src_lo = k == 0 ? position : 0;
    const int src_hi = n;
    reach_copy_kernel<<<dim3(wgs_words), 256, 0, stream>>>(nxt, cur, nwords);
    const unsigned gx = (unsigned)((src_hi - src_lo + kTokensPerWg - 1) / kTokensPerWg);
    reach_step_kernel<<<dim3(gx, nwin), 256, 0, stream>>>(layers[k], n, src_lo, src_hi, cur, nxt);
    if (counts)
      reach_popcount_kernel<<<dim3(std::min(wgs_words, 1024u)), 256, 0, stream>>>(nxt, nwords,
                                                                                counts + k);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    std::swap(cur, nxt);
  }
  return hipSuccess;
}

}  // namespace esa
