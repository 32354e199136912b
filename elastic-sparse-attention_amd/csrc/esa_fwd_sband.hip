// Staged-band forward over the elastic pattern (gfx950), prefill rows: the
// band kernel's per-band arithmetic over K/V that a workgroup stages once.
//
// Replaces the forward branch of the reference's per-token Triton kernel
// (elastic_sparse_attention.py:117-166) for query positions 0 .. q_len - 1,
// like band_fwd_kernel (esa_fwd_band.hip), for shapes where rows are short:
// there the 16-key bands of neighbouring row groups overlap, and gathering
// every band separately (band_fwd_kernel: 16 keys per entry and 16 rows,
// through the texture path) moves two to three times the bytes the rows'
// keys span.  Here a workgroup of eight waves takes 128 consecutive rows of
// one (batch, head); the keys their bands touch form one ascending range,
// which is streamed once through a ring of 256 K and V rows in LDS (16
// chunks of 16 keys, XOR-swizzled as in the band kernel), 64 keys per round
// while the next 64 load.  Each wave walks its 16 rows' 16-key windows in
// entry order -- one per index-list entry, two for a band wider than 16
// keys -- as far as the resident range reaches, then the workgroup meets at
// a barrier and the ring advances.  Windows rise with the entry (a row's
// keys rise with j, and a band moves by at most a key or two per row), so
// every window is resident in some round.
//
// Per window pair and wave, exactly the band kernel's steps: S^T = K Q^T on
// 16x16x32 MFMA with the window's 16 K rows read from the ring, the lane
// holding each row's key keeps its score, online softmax once per pair, and
// O^T += V^T P^T over the two windows' 32 keys (V^T read transposed from the
// ring).  Each row's key of an entry lies in exactly one of its windows, so
// no key counts twice.  Operand layouts: esa_band.hpp.
#include "esa_band.hpp"

namespace esa {

constexpr int kSbWaves = 8;          // waves per workgroup (16 rows each)
constexpr int kSbRows = 16 * kSbWaves;
constexpr int kRingRows = 256;       // K (and V) rows held in LDS
constexpr int kChunk = 16;           // keys per ring chunk
constexpr int kAdvance = 4;          // chunks the ring advances per round
constexpr int kProcRows = kRingRows - kAdvance * kChunk;  // keys resident for processing

template <int D, Elem E>
__global__ __launch_bounds__(64 * kSbWaves, 1) void sband_fwd_kernel(BandArgs A) {
  using C = BandCfg<D>;
  using M = MmaT<E>;
  using V8 = typename M::v8;
  __shared__ __attribute__((aligned(1024))) uint16_t kring[kRingRows * D];
  __shared__ __attribute__((aligned(1024))) uint16_t vring[kRingRows * D];
  // per wave: each row's key of entry j as an offset from the band's first
  // key (0xff: no key), and the band descriptors lo | W << 24
  __shared__ uint8_t koff_all[kSbWaves][64][16];
  __shared__ int info_all[kSbWaves][64];

  // ---- item: XCD x takes the contiguous range [x per, (x + 1) per), so the
  // neighbouring row blocks of a head (whose keys mostly coincide) share an L2
  const int bid = blockIdx.x;
  const int item = (bid & 7) * A.per_xcd + (bid >> 3);
  if (item >= A.n_groups) return;
  const int bh = item / A.ng, blk = item % A.ng;
  const int h = bh % A.H, b = bh / A.H;
  const int kvh = h / A.groups;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, q = lane >> 4;
  const int i0 = blk * kSbRows;
  const int i = i0 + 16 * wave + n;  // this lane's query row
  const bool row_ok = i < A.q_len;
  uint8_t (*koff)[16] = koff_all[wave];
  int* info_w = info_all[wave];

  // ---- Q as the B operand: row n, dims 32 s + 8 q .. + 8 for k-step s
  V8 qop[C::NS];
  {
    const uint16_t* qrow = A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)i * A.qss;
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row_ok) raw = *(const u32x4*)(qrow + 32 * s + 8 * q);
      qop[s] = __builtin_bit_cast(V8, raw);
    }
  }

  // ---- this row's keys of entries 16 q .. 16 q + 15 and the wave's band
  // descriptors, kept in LDS so the walk below can index entries at run time
  {
    int kreg[16], info[16];
    band_rows(A.pc, h, i, row_ok, q, 0, kreg, info);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int lo = info[r] & 0xffffff;
      koff[16 * q + r][n] = kreg[r] < 0 ? (uint8_t)0xff : (uint8_t)(kreg[r] - lo);
      if (n == 0) info_w[16 * q + r] = info[r];
    }
  }

  __syncthreads();  // every wave's koff / info written
  // ---- the workgroup's key range: the smallest first key and the largest
  // last key of any band of its waves (512 descriptors), the start aligned
  // down to a chunk
  int k_lo, k_hi;
  {
    int lo = 0x7fffffff, hi = -1;
#pragma unroll
    for (int t = 0; t < kSbWaves * 64 / 64; ++t) {
      const int bi = (&info_all[0][0])[64 * t + lane];
      const int wdt = (int)((uint32_t)bi >> 24);
      if (wdt > 0) {
        lo = min(lo, bi & 0xffffff);
        hi = max(hi, (bi & 0xffffff) + wdt - 1);
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      lo = min(lo, __shfl_xor(lo, off, 64));
      hi = max(hi, __shfl_xor(hi, off, 64));
    }
    k_lo = __builtin_amdgcn_readfirstlane(hi < 0 ? 0 : lo & ~(kChunk - 1));
    k_hi = __builtin_amdgcn_readfirstlane(hi < 0 ? 0 : hi);
  }
  // rounds: round r holds keys [k_lo + 64 r, k_lo + 64 r + kProcRows) for
  // processing; a window [c0, c0 + 16) needs c0 + 16 within that, and no
  // window starts past k_hi
  const int span = k_hi + kChunk - (k_lo + kProcRows);
  const int n_rounds = span <= 0 ? 1 : 1 + (span + kAdvance * kChunk - 1) / (kAdvance * kChunk);

  // ---- staging: chunk c (keys k_lo + 16 c ..) -> ring rows 16 (c % 16) ..
  // through buffer resources over this (batch, kv head)'s rows (rows at or
  // past kv_len read as zeros).  Wave w loads matrix w & 1 (K, V) of chunk
  // w / 2 of each four-chunk batch; DMA t, lane l fills ring row 4 t + l /
  // CPR (D = 128) of the chunk, physical 16-byte piece l % CPR.
  const bool is_v = (wave & 1) != 0;
  const int my_chunk = wave >> 1;  // 0 .. 3 within a batch
  const int ss2 = is_v ? (int)A.vss * 2 : (int)A.kss * 2;
  const uint16_t* const src =
      is_v ? A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh
           : A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)src, (short)0, (int)((int64_t)A.q_len * ss2), 0x00020000);
  int dofs[C::VLOADS];
#pragma unroll
  for (int t = 0; t < C::VLOADS; ++t) {
    const int R = (64 * t + lane) / C::CPR, pc = lane % C::CPR;
    dofs[t] = R * ss2 + 16 * (is_v ? vswz<D>(R, pc) : kswz<D>(R, pc));
  }
  uint16_t* const ring = is_v ? vring : kring;
  // (every chunk is loaded, past the last key too, so no window reads a ring
  // row that holds anything but loaded K / V rows or zeros)
  auto issue_batch = [&](int c_first) {
    const int c = c_first + my_chunk;
    const int key0 = k_lo + kChunk * c;
    uint16_t* dst = ring + (c % (kRingRows / kChunk)) * kChunk * D;
#pragma unroll
    for (int t = 0; t < C::VLOADS; ++t)
      load_lds16(rs, dst + 512 * t, dofs[t], key0 * ss2);
  };

  // ---- the walk: this wave's windows in entry order.  Window (j, m) covers
  // keys lo_j + 16 m .. + 15 (the band's keys past lo_j + W_j - 1 are unused
  // or read as zeros); it is resident in round r when its last key lies below
  // k_lo + 64 r + kProcRows.
  const float scale = A.scale_log2;
  float m_run = -INFINITY, l_run = 0.f, n_run = 0.f;
  f32x4 oacc[C::NV];
#pragma unroll
  for (int s = 0; s < C::NV; ++s) oacc[s] = f32x4{};

  // ring byte addresses of the window at first key c0: K operand rows
  // (lane row n, dims 32 s + 8 q), V^T operand rows (4 q + x / 4)
  auto k_addr = [&](int c0, int s) {
    const int rr = (c0 - k_lo + n) & (kRingRows - 1);
    return rr * C::ROWB + 16 * kswz<D>(rr, 4 * s + q);
  };
  auto v_addr = [&](int c0, int s) {
    const int R = 4 * q + (n >> 2);
    const int rr = (c0 - k_lo + R) & (kRingRows - 1);
    const int dim0 = C::CW * (n & 3) + 4 * s;
    return rr * C::ROWB + 16 * vswz<D>(rr, dim0 >> 3) + 2 * (dim0 & 7);
  };
  auto scores = [&](int c0) {
    V8 kb[C::NS];
#pragma unroll
    for (int s = 0; s < C::NS; ++s) kb[s] = *(const V8*)((const char*)kring + k_addr(c0, s));
    f32x4 sacc = M::mfma16(kb[0], qop[0], f32x4{});
#pragma unroll
    for (int s = 1; s < C::NS; ++s) sacc = M::mfma16(kb[s], qop[s], sacc);
    return sacc;
  };
  // this row's scaled score (log2 units) in the window at c0 (key: the row's
  // key of the entry, -1 for none), the same in the row's 4 lanes; -inf when
  // the row has no key there.  has / e: this lane holds the key, at register e.
  auto pick = [&](const f32x4& sacc, int key, int c0, bool& has, int& e) -> float {
    const int d = key - c0;
    has = key >= 0 && (uint32_t)d < 16u && (d >> 2) == q;
    e = d & 3;
    const float s01 = (e & 1) ? sacc[1] : sacc[0];
    const float s23 = (e & 1) ? sacc[3] : sacc[2];
    const float s = (e & 2) ? s23 : s01;
    return row4_max(has ? s * scale : -INFINITY);
  };
  // online softmax over two windows' scores (one running-max update per pair)
  // -> P words (the input type at register e of the lane holding the key)
  auto pair_softmax = [&](float xa, bool ha, int ea, float xb, bool hb, int eb, uint64_t& pa,
                          uint64_t& pb) {
    const float xm = fmaxf(xa, xb);
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float ra = xa - m_use, rb = xb - m_use;
    const float rm = xm - m_use;
    const bool grow = m_run == -INFINITY ? xm != -INFINITY : rm > kRescaleSlack;
    if (wave_any(grow)) {
      const float delta = grow ? rm : 0.f;
      const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - (m_use + delta)) : 1.0f;
      l_run *= alpha;
      n_run *= alpha;
#pragma unroll
      for (int v = 0; v < C::NV; ++v) oacc[v] *= alpha;
      m_run = grow ? m_use + delta : m_run;
      ra -= delta;
      rb -= delta;
    }
    const float p0 = __builtin_amdgcn_exp2f(ra);
    const float p1 = __builtin_amdgcn_exp2f(rb);
    l_run += p0;
    l_run += p1;
    const uint32_t b0 = (uint32_t)M::bits(p0);
    const uint32_t b1 = (uint32_t)M::bits(p1);
    n_run += M::val(b0);
    n_run += M::val(b1);
    pa = ha ? ((uint64_t)b0 << (16 * ea)) : 0ull;
    pb = hb ? ((uint64_t)b1 << (16 * eb)) : 0ull;
  };
  auto pv = [&](int ca, int cb, uint64_t pa, uint64_t pb) {
    s16x4 ta[C::NV], tb[C::NV];
#pragma unroll
    for (int s = 0; s < C::NV; ++s) {
      ta[s] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)((const char*)vring + v_addr(ca, s)));
      tb[s] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)((const char*)vring + v_addr(cb, s)));
    }
    const u32x4 pq = {(uint32_t)pa, (uint32_t)(pa >> 32), (uint32_t)pb, (uint32_t)(pb >> 32)};
    const V8 pop = __builtin_bit_cast(V8, pq);
#pragma unroll
    for (int s = 0; s < C::NV; ++s) {
      const s16x4 vv[2] = {ta[s], tb[s]};
      oacc[s] = M::mfma16(__builtin_bit_cast(V8, vv), pop, oacc[s]);
    }
  };

  // the wave's window cursor (uniform): entry j, sub-window m; entries with
  // no key in any of the wave's rows (W = 0) are skipped
  int cj = 0, cm = 0;
  auto band_of = [&](int j) { return __builtin_amdgcn_readfirstlane(info_w[j]); };
  // next window at or after (j, m) -> (j, m), first key c0; false when none
  auto seek = [&](int& j, int& m, int& c0) -> bool {
    while (j < 64) {
      const int bi = band_of(j);
      const int wdt = (int)((uint32_t)bi >> 24);
      if (m * kChunk < wdt) {
        c0 = (bi & 0xffffff) + kChunk * m;
        return true;
      }
      ++j;
      m = 0;
    }
    return false;
  };
  auto row_key = [&](int j, int c0, int m) {
    const int off = koff[j][n];
    const int lo = c0 - kChunk * m;
    return off == 0xff ? -1 : lo + off;
  };

  // prologue: all 16 chunks of the ring (4 batches)
#pragma unroll
  for (int c = 0; c < kRingRows / kChunk; c += kAdvance) issue_batch(c);
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();  // the ring is in LDS (every wave's DMAs)

  // round r processes chunks 4 r .. 4 r + 11; at its end the chunks 4 r + 12
  // .. 4 r + 15 loaded during it are waited for, and 4 r .. 4 r + 3 make room
  // for 4 r + 16 .. 4 r + 19
  for (int r = 0; r < n_rounds; ++r) {
    const int lim = k_lo + kAdvance * kChunk * r + kProcRows;  // first key not resident
    for (;;) {
      int ja = cj, ma = cm, ca = 0;
      if (!seek(ja, ma, ca) || ca + kChunk > lim) break;
      int jb = ja, mb = ma + 1, cb = 0;
      const bool has_b = seek(jb, mb, cb);
      if (has_b && cb + kChunk > lim) break;  // wait for the pair to be resident
      const int keya = row_key(ja, ca, ma);
      const int keyb = has_b ? row_key(jb, cb, mb) : -1;
      const f32x4 sa = scores(ca);
      const f32x4 sb = has_b ? scores(cb) : f32x4{};
      bool ha, hb;
      int ea, eb;
      const float xa = pick(sa, keya, ca, ha, ea);
      const float xb = has_b ? pick(sb, keyb, cb, hb, eb) : -INFINITY;
      if (!has_b) {
        hb = false;
        eb = 0;
      }
      uint64_t pa, pbw;
      pair_softmax(xa, ha, ea, xb, hb, eb, pa, pbw);
      // a missing second window contributes p = 0 against the first's V rows
      pv(ca, has_b ? cb : ca, pa, pbw);
      if (has_b) {
        cj = jb;
        cm = mb + 1;
      } else {
        cj = ja;
        cm = ma + 1;
      }
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();  // every wave is done with the oldest four chunks
    if (r + 1 < n_rounds) issue_batch(kRingRows / kChunk + kAdvance * r);
  }

  // ---- epilogue: lane (n, q) holds O^T[dim][row n] for dims CW q .. CW q + CW
  if (row_ok) {
    const float inv = n_run > 0.f ? 1.f / n_run : 0.f;
    uint16_t* orow = A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)i * A.oss;
#pragma unroll
    for (int t = 0; t < C::NV / 2; ++t) {
      V8 ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ov[e] = (typename M::s)(oacc[2 * t][e] * inv);
        ov[4 + e] = (typename M::s)(oacc[2 * t + 1][e] * inv);
      }
      *(V8*)(orow + C::CW * q + 8 * t) = ov;
    }
    if (A.lse && q == 0) {
      const float lse = l_run > 0.f ? (m_run + __log2f(l_run)) * 0.69314718055994530942f
                                    : -INFINITY;
      A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + i] = lse;
    }
  }
}

namespace {

template <Elem E>
void launch_sband_elem(const BandArgs& a, int head_dim, dim3 grid, hipStream_t stream) {
  if (head_dim == 128)
    sband_fwd_kernel<128, E><<<grid, 64 * kSbWaves, 0, stream>>>(a);
  else
    sband_fwd_kernel<64, E><<<grid, 64 * kSbWaves, 0, stream>>>(a);
}

}  // namespace

int sband_rows() { return kSbRows; }

hipError_t launch_sband_fwd(const BandArgs& a, int head_dim, hipStream_t stream) {
  if (a.n_groups <= 0) return hipSuccess;
  const dim3 grid((unsigned)(8 * a.per_xcd));
  if (a.elem == (int)Elem::f16)
    launch_sband_elem<Elem::f16>(a, head_dim, grid, stream);
  else
    launch_sband_elem<Elem::bf16>(a, head_dim, grid, stream);
  return hipGetLastError();
}

}  // namespace esa
