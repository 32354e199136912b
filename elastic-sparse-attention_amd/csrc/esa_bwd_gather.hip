// Gather backward (gfx950): dQ, dK and dV for any index source (explicit
// index lists, the elastic pattern at positions, float32 / bfloat16 /
// float16, any head_dim that is a multiple of 4 up to 256).
//
// Replaces the backward branch of the reference's Triton kernel
// (elastic_sparse_attention.py:168-233) as ElasticSparseAttentionFunction
// .backward launches it (:299-339), without its float atomics:
//
//   bwd_rows_kernel   one wave per (batch, head, query row): delta = dO . O,
//                     then per entry j (lane j): s = q . k_j * scale,
//                     p = exp(s - lse) (valid entries), dp = dO . v_j,
//                     dS = p (m_j dp - delta) with m_j the dropout factor,
//                     dQ = scale * sum_j dS_j k_j; each entry's dV
//                     coefficient m_j p and dK coefficient scale * dS go to
//                     the workspace (0 for an entry that is masked or whose
//                     key lies outside [0, kv_len): the Triton kernel's
//                     atomics skip those, :209-213, :226-228).  A row
//                     with a non-finite delta and an entry it does not
//                     attend gets a NaN dQ, as the Triton kernel's
//                     (0 - delta) * 0 term for that entry gives it.
//   bwd_sort_keys     key of each entry: kv_head * kv_len + key for a valid
//                     in-range entry, else a sentinel past every key.
//   radix sort        a stable LSD radix sort of (key, entry id), 8 bits per
//                     pass (per-tile digit histograms, an exclusive scan of
//                     them, then a scatter ranked by wave ballots): each
//                     key's entries end up contiguous, in entry order.
//   bwd_segments      the start of each (kv head, key) in the sorted order.
//   bwd_kv_kernel     one wave per (batch, kv head, key): dK = sum of
//                     coefficient * q row and dV = sum of coefficient * dO
//                     row over the key's entries, in entry order.
//
// Every gradient element is summed by one wave in a fixed order, so two
// runs agree bit for bit.  The index lists do not depend on the batch, so
// the sort serves every batch element.
#include "esa_gather.hpp"

namespace esa {

namespace {

template <Elem E, bool PATTERN>
__global__ __launch_bounds__(256) void bwd_rows_kernel(GatherBwdArgs A) {
  using T = typename ElemT<E>::T;
  __shared__ float qs_all[4][256];
  __shared__ float dos_all[4][256];
  __shared__ float ds_all[4][64];
  __shared__ int ks_all[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = blockIdx.x * 4 + wave;
  const int h = blockIdx.y, b = blockIdx.z;
  if (r >= A.q_len) return;  // whole wave leaves; no block-level barrier below
  const int kvh = h / A.groups;
  const int D = A.D;
  float* qs = qs_all[wave];
  float* dos = dos_all[wave];
  float* dsl = ds_all[wave];
  int* ksl = ks_all[wave];

  const T* qrow = (const T*)A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)r * A.qss;
  const T* orow = (const T*)A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)r * A.oss;
  const T* dorow =
      (const T*)A.dout + (int64_t)b * A.dosb + (int64_t)h * A.dosh + (int64_t)r * A.doss;
  float dl = 0.f;
  for (int d = lane; d < D; d += 64) {
    qs[d] = ElemT<E>::load(qrow + d);
    const float g = ElemT<E>::load(dorow + d);
    dos[d] = g;
    dl += g * ElemT<E>::load(orow + d);
  }
  const float delta = wave_sum(dl);  // dO . O (the output the forward stored)
  wave_sync_lds();

  const T* kbase = (const T*)A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh;
  const T* vbase = (const T*)A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh;
  RowEntries row;
  row.init<PATTERN>(A.src, h, r);
  const float lse = A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + r];
  const int w = A.src.w;
  const int64_t e0 = ((int64_t)h * A.q_len + r) * w;  // entry id of (h, r, 0)
  float* cp = A.cp + (int64_t)b * A.E;
  float* cs = A.cs + (int64_t)b * A.E;

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  bool dead = false;
  for (int c0 = 0; c0 < w; c0 += 64) {
    const int j = c0 + lane;
    bool valid = false;
    int64_t key = 0;
    if (j < w) row.entry<PATTERN>(A.src, h, r, j, valid, key);
    const bool in_range = key >= 0 && key < A.kv_len;
    const bool live = valid && in_range && !row.bad_pos;
    dead |= j < w && !live;
    float dsc = 0.f, pc = 0.f;
    if (live) {
      const float s = row_dot<E>(qs, kbase + key * A.kss, D) * A.sm_scale;
      const float dp = row_dot<E>(dos, vbase + key * A.vss, D);
      const float p = expf(s - lse);
      const float keep = drop_factor(A.drop, b, h, r, j, A.H, A.q_len, w);
      pc = keep * p;
      dsc = p * (keep * dp - delta) * A.sm_scale;
    }
    if (j < w) {
      cp[e0 + j] = pc;
      cs[e0 + j] = dsc;
    }
    dsl[lane] = dsc;
    ksl[lane] = live ? (int)key : -1;
    wave_sync_lds();
    const int nj = min(64, w - c0);
    for (int jj = 0; jj < nj; ++jj) {
      const float g = dsl[jj];
      const int kj = ksl[jj];
      if (kj >= 0) {
        const T* kr = kbase + (int64_t)kj * A.kss;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = lane + 64 * e;
          if (d < D) acc[e] += g * ElemT<E>::load(kr + d);
        }
      }
    }
    wave_sync_lds();
  }
  T* dqrow = (T*)A.dq + (int64_t)b * A.dqsb + (int64_t)h * A.dqsh + (int64_t)r * A.dqss;
  // an entry the row does not attend (masked, or a key outside [0, kv_len))
  // adds dS * 0 in the Triton kernel with dS = p (0 - delta) scale (:202-221):
  // NaN throughout when delta is not finite
  const bool all_nan = row.bad_pos || (__builtin_amdgcn_ballot_w64(dead) != 0 && !__builtin_isfinite(delta));
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int d = lane + 64 * e;
    if (d < D) ElemT<E>::store(dqrow + d, all_nan ? __builtin_nanf("") : acc[e]);
  }
}

// Sort keys of every entry (batch-independent): kv_head * kv_len + key of a
// valid entry with a key in [0, kv_len), else the sentinel Hkv * kv_len.
template <bool PATTERN>
__global__ __launch_bounds__(256) void bwd_sort_keys(GatherBwdArgs A) {
  const int w = A.src.w;
  const uint32_t sentinel = (uint32_t)A.Hkv * (uint32_t)A.kv_len;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < A.E;
       e += (int64_t)gridDim.x * 256) {
    const int j = (int)(e % w);
    const int64_t hr = e / w;
    const int r = (int)(hr % A.q_len), h = (int)(hr / A.q_len);
    RowEntries row;
    row.init<PATTERN>(A.src, h, r);
    bool valid = false;
    int64_t key = 0;
    row.entry<PATTERN>(A.src, h, r, j, valid, key);
    const bool live = valid && key >= 0 && key < A.kv_len && !row.bad_pos;
    A.keys_in[e] = live ? (uint32_t)(h / A.groups) * (uint32_t)A.kv_len + (uint32_t)key : sentinel;
    A.vals_in[e] = (uint32_t)e;
  }
}

// seg[g] = the first sorted position whose key is >= g, g = 0 .. Hkv * kv_len
__global__ __launch_bounds__(256) void bwd_segments(GatherBwdArgs A) {
  const int64_t n_keys = (int64_t)A.Hkv * A.kv_len;
  for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g <= n_keys;
       g += (int64_t)gridDim.x * 256) {
    int64_t lo = 0, hi = A.E;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if ((int64_t)A.keys_out[mid] < g)
        lo = mid + 1;
      else
        hi = mid;
    }
    A.seg[g] = (int32_t)lo;
  }
}

// dK and dV of one (batch, kv head, key): its entries in sorted (entry id)
// order, four at a time (their q / dO rows loaded together), lanes over D.
template <Elem E>
__global__ __launch_bounds__(256) void bwd_kv_kernel(GatherBwdArgs A) {
  using T = typename ElemT<E>::T;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int key = blockIdx.x * 4 + wave;
  const int kvh = blockIdx.y, b = blockIdx.z;
  if (key >= A.kv_len) return;
  const int D = A.D;
  const int w = A.src.w;
  const int64_t g = (int64_t)kvh * A.kv_len + key;
  const int i0 = A.seg[g], i1 = A.seg[g + 1];
  const float* cp = A.cp + (int64_t)b * A.E;
  const float* cs = A.cs + (int64_t)b * A.E;
  float dk[4] = {0.f, 0.f, 0.f, 0.f}, dv[4] = {0.f, 0.f, 0.f, 0.f};
  constexpr int U = 4;
  for (int i = i0; i < i1; i += U) {
    float qv[U][4], gv[U][4], c_s[U], c_p[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool in = i + u < i1;
      const uint32_t e = in ? A.vals_out[i + u] : A.vals_out[i0];
      const int64_t hr = e / (uint32_t)w;
      const int r = (int)(hr % A.q_len), h = (int)(hr / A.q_len);
      c_s[u] = in ? cs[e] : 0.f;
      c_p[u] = in ? cp[e] : 0.f;
      const T* qrow = (const T*)A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)r * A.qss;
      const T* dorow =
          (const T*)A.dout + (int64_t)b * A.dosb + (int64_t)h * A.dosh + (int64_t)r * A.doss;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d = lane + 64 * q;
        // (a padding slot's row counts 0, not 0 times that row)
        qv[u][q] = in && d < D ? ElemT<E>::load(qrow + d) : 0.f;
        gv[u][q] = in && d < D ? ElemT<E>::load(dorow + d) : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        dk[q] += c_s[u] * qv[u][q];
        dv[q] += c_p[u] * gv[u][q];
      }
    }
  }
  T* dkrow = (T*)A.dk + (int64_t)b * A.dksb + (int64_t)kvh * A.dksh + (int64_t)key * A.dkss;
  T* dvrow = (T*)A.dv + (int64_t)b * A.dvsb + (int64_t)kvh * A.dvsh + (int64_t)key * A.dvss;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int d = lane + 64 * q;
    if (d < D) {
      ElemT<E>::store(dkrow + d, dk[q]);
      ElemT<E>::store(dvrow + d, dv[q]);
    }
  }
}

unsigned grid_for(int64_t n) {
  const int64_t blocks = (n + 255) / 256;
  return (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

// ---------------------------------------------------------------------------
// Stable LSD radix sort of (uint32 key, uint32 value) pairs, 8 bits a pass.
// A tile is 4096 pairs: wave w of a 256-thread block owns tile positions
// [1024 w, 1024 (w + 1)), item i and lane l holding position 1024 w + 64 i + l,
// so (wave, item, lane) order is the input order.
constexpr int kSortTile = 4096;
constexpr int kScanChunk = 2048;

// hist[d * nb + blk] = pairs of tile blk whose digit is d
__global__ __launch_bounds__(256) void radix_hist(const uint32_t* __restrict__ keys, int64_t n,
                                                  int shift, int nb, int32_t* __restrict__ hist) {
  __shared__ int cnt[256];
  const int blk = blockIdx.x;
  cnt[threadIdx.x] = 0;
  __syncthreads();
  const int64_t t0 = (int64_t)blk * kSortTile;
  for (int i = threadIdx.x; i < kSortTile; i += 256) {
    const int64_t x = t0 + i;
    if (x < n) atomicAdd(&cnt[(keys[x] >> shift) & 255u], 1);
  }
  __syncthreads();
  hist[(int64_t)threadIdx.x * nb + blk] = cnt[threadIdx.x];
}

// exclusive scan of 256 per-thread values over the block (Hillis-Steele in
// LDS); returns the thread's exclusive prefix and the block total in *total
__device__ __forceinline__ int block_exclusive_scan(int v, int* buf, int* total) {
  const int t = threadIdx.x;
  buf[t] = v;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int add = t >= off ? buf[t - off] : 0;
    __syncthreads();
    buf[t] += add;
    __syncthreads();
  }
  *total = buf[255];
  const int incl = buf[t];
  __syncthreads();
  return incl - v;
}

// parts[c] = sum of chunk c of x (kScanChunk entries)
__global__ __launch_bounds__(256) void scan_chunk_sums(const int32_t* __restrict__ x, int64_t n,
                                                       int32_t* __restrict__ parts) {
  __shared__ int buf[256];
  const int64_t c0 = (int64_t)blockIdx.x * kScanChunk;
  int v = 0;
  for (int i = threadIdx.x; i < kScanChunk; i += 256)
    if (c0 + i < n) v += x[c0 + i];
  int total = 0;
  block_exclusive_scan(v, buf, &total);
  if (threadIdx.x == 0) parts[blockIdx.x] = total;
}

// exclusive scan of the chunk sums in place (one block)
__global__ __launch_bounds__(256) void scan_parts(int32_t* __restrict__ parts, int np) {
  __shared__ int buf[256];
  int carry = 0;
  for (int base = 0; base < np; base += 256) {
    const int i = base + threadIdx.x;
    const int v = i < np ? parts[i] : 0;
    int total = 0;
    const int ex = block_exclusive_scan(v, buf, &total);
    if (i < np) parts[i] = carry + ex;
    carry += total;
  }
}

// out = exclusive scan of x: each chunk scanned in the block (eight
// consecutive entries per thread), plus its chunk's prefix
__global__ __launch_bounds__(256) void scan_apply(const int32_t* __restrict__ x, int64_t n,
                                                  const int32_t* __restrict__ parts,
                                                  int32_t* __restrict__ out) {
  __shared__ int buf[256];
  constexpr int PER = kScanChunk / 256;
  const int64_t c0 = (int64_t)blockIdx.x * kScanChunk + (int64_t)threadIdx.x * PER;
  int v[PER];
  int sum = 0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    v[k] = c0 + k < n ? x[c0 + k] : 0;
    sum += v[k];
  }
  int total = 0;
  int run = block_exclusive_scan(sum, buf, &total) + parts[blockIdx.x];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    if (c0 + k < n) out[c0 + k] = run;
    run += v[k];
  }
}

// Scatter of one pass: a pair goes to offs[d * nb + blk] + (pairs of digit d
// in earlier waves of the tile) + (pairs of digit d before it in its wave).
// Ranks within a wave come from eight ballots per item (the lanes sharing
// the pair's digit) and per-wave running digit counts in LDS.
__global__ __launch_bounds__(256) void radix_scatter(const uint32_t* __restrict__ kin,
                                                     const uint32_t* __restrict__ vin, int64_t n,
                                                     int shift, int nb,
                                                     const int32_t* __restrict__ offs,
                                                     uint32_t* __restrict__ kout,
                                                     uint32_t* __restrict__ vout) {
  __shared__ int cnt[4][256];
  constexpr int ITEMS = kSortTile / 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int blk = blockIdx.x;
  for (int i = threadIdx.x; i < 4 * 256; i += 256) (&cnt[0][0])[i] = 0;
  __syncthreads();
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
  const int64_t p0 = (int64_t)blk * kSortTile + (int64_t)wave * (64 * ITEMS);
  uint32_t key[ITEMS], val[ITEMS];
  int rank[ITEMS];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int64_t x = p0 + (int64_t)it * 64 + lane;
    const bool ok = x < n;
    key[it] = ok ? kin[x] : 0u;
    val[it] = ok ? vin[x] : 0u;
    const uint32_t d = (key[it] >> shift) & 255u;
    uint64_t peers = __builtin_amdgcn_ballot_w64(ok);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const uint64_t bal = __builtin_amdgcn_ballot_w64(((d >> bit) & 1u) != 0u);
      peers &= ((d >> bit) & 1u) ? bal : ~bal;
    }
    const int base = cnt[wave][d];
    rank[it] = base + __builtin_popcountll(peers & below);
    wave_sync_lds();
    // the lowest lane of each digit group advances that digit's count
    if (ok && (peers & below) == 0ull) cnt[wave][d] = base + __builtin_popcountll(peers);
    wave_sync_lds();
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int64_t x = p0 + (int64_t)it * 64 + lane;
    if (x >= n) continue;
    const uint32_t d = (key[it] >> shift) & 255u;
    int before = 0;
    for (int w2 = 0; w2 < wave; ++w2) before += cnt[w2][d];
    const int64_t dst = (int64_t)offs[(int64_t)d * nb + blk] + before + rank[it];
    kout[dst] = key[it];
    vout[dst] = val[it];
  }
}

// Sorts (A.keys_in, A.vals_in) over the low key_bits bits; returns, through
// *keys / *vals, the buffers holding the result (the pair buffers alternate
// by pass).
hipError_t radix_sort(const GatherBwdArgs& A, const uint32_t** keys, const uint32_t** vals,
                      hipStream_t stream) {
  const int64_t n = A.E;
  const int nb = (int)((n + kSortTile - 1) / kSortTile);
  const int64_t nh = (int64_t)256 * nb;
  const int np = (int)((nh + kScanChunk - 1) / kScanChunk);
  uint32_t* ka = A.keys_in;
  uint32_t* va = A.vals_in;
  uint32_t* kb = A.keys_out;
  uint32_t* vb = A.vals_out;
  for (int shift = 0; shift < A.key_bits; shift += 8) {
    radix_hist<<<nb, 256, 0, stream>>>(ka, n, shift, nb, A.hist);
    scan_chunk_sums<<<np, 256, 0, stream>>>(A.hist, nh, A.parts);
    scan_parts<<<1, 256, 0, stream>>>(A.parts, np);
    scan_apply<<<np, 256, 0, stream>>>(A.hist, nh, A.parts, A.offs);
    radix_scatter<<<nb, 256, 0, stream>>>(ka, va, n, shift, nb, A.offs, kb, vb);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    uint32_t* t = ka; ka = kb; kb = t;
    t = va; va = vb; vb = t;
  }
  *keys = ka;
  *vals = va;
  return hipSuccess;
}

template <Elem E>
hipError_t launch_elem(const GatherBwdArgs& a, bool pattern, hipStream_t stream) {
  GatherBwdArgs s = a;
  hipError_t e = hipSuccess;
  if (a.E > 0) {
    const dim3 rows_grid((unsigned)((a.q_len + 3) / 4), (unsigned)a.H, (unsigned)a.B);
    if (pattern)
      bwd_rows_kernel<E, true><<<rows_grid, 256, 0, stream>>>(a);
    else
      bwd_rows_kernel<E, false><<<rows_grid, 256, 0, stream>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (pattern)
      bwd_sort_keys<true><<<grid_for(a.E), 256, 0, stream>>>(a);
    else
      bwd_sort_keys<false><<<grid_for(a.E), 256, 0, stream>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t* sk = nullptr;
    const uint32_t* sv = nullptr;
    e = radix_sort(a, &sk, &sv, stream);
    if (e != hipSuccess) return e;
    s.keys_out = const_cast<uint32_t*>(sk);
    s.vals_out = const_cast<uint32_t*>(sv);
  }
  // with no entries every segment is empty and dK = dV = 0
  bwd_segments<<<grid_for((int64_t)a.Hkv * a.kv_len + 1), 256, 0, stream>>>(s);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 kv_grid((unsigned)((a.kv_len + 3) / 4), (unsigned)a.Hkv, (unsigned)a.B);
  bwd_kv_kernel<E><<<kv_grid, 256, 0, stream>>>(s);
  return hipGetLastError();
}

}  // namespace

void gather_bwd_sort_sizes(int64_t n, int64_t* hist_ints, int64_t* part_ints) {
  const int64_t nb = (n + kSortTile - 1) / kSortTile;
  *hist_ints = 256 * nb;
  *part_ints = (256 * nb + kScanChunk - 1) / kScanChunk;
}

hipError_t launch_gather_bwd(const GatherBwdArgs& a, bool pattern, hipStream_t stream) {
  if (a.B <= 0 || a.H <= 0 || a.kv_len <= 0) return hipSuccess;
  switch ((Elem)a.elem) {
    case Elem::f32: return launch_elem<Elem::f32>(a, pattern, stream);
    case Elem::bf16: return launch_elem<Elem::bf16>(a, pattern, stream);
    default: return launch_elem<Elem::f16>(a, pattern, stream);
  }
}

}  // namespace esa
