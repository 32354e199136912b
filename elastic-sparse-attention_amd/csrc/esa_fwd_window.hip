// Sliding-window forward: the elastic pattern at interpolation weight 0
// (layer 0) on gfx950, prefill rows.
//
// At weight 0 the recipe of elastic_sparse_attention.py:482-535 gives row i
// the window start st = i + 1 - w (clamped at 0) and spacing 1, so entry j's
// key is st + j and the row attends exactly the keys max(0, i - w + 1) .. i
// (every head alike: both interpolated terms equal st + j).  A 16-row group
// [r0, r0 + 16) then needs only the keys [max(0, r0 - w + 1), r0 + 16): at
// most w + 15, five 16-key chunks at w = 64, where the band kernel would
// gather 64 bands of 16 keys (all but 15 keys of each shared with the next).
//
// One wave per group, as in band_fwd_kernel (whose slot layouts, swizzles,
// DMA staging and MFMA forms this kernel shares; esa_band.hpp):
//   per chunk pair (32 keys): both chunks' K and V rows reach LDS by
//   buffer_load ... lds (rows past the group's last key are not loaded);
//   S^T = K Q^T (D/32 x v_mfma_f32_16x16x32 per chunk, Q in registers);
//   each lane (row n, lane group q) holds keys 4 q .. 4 q + 3 of both
//   chunks for its row and keeps the ones in the row's window (a select:
//   masked scores never mix with a non-finite K value); one online-softmax
//   update per pair over those 8 scores and the row's 4 lanes; O^T += V^T
//   P^T with the pair's 32 keys as one k-step (D/16 MFMAs, V^T read with
//   ds_read_b64_tr_b16).
// The next pair's K and V are requested once this pair's operands are in
// registers (the band kernel's early refill order).  Groups go to the XCDs
// in contiguous ranges (rows ascending within a head), so consecutive groups
// of one head, which share all but 32 of their keys, run on one L2.  The
// next group's pair p is this group's pair p + 1, so each group starts at
// pair (-group) mod n_pairs and wraps around: the groups sharing a pair load
// it at the same step instead of one to two pairs apart, by which time it had
// often left L2 (layer 0 forward at B=1 H=32 L=8192 0.059 -> 0.050 ms,
// L=32768 -2%).
//
// POS: rows at positions A.positions[r] (a chunked prefill's cache_position).
// A group whose rows sit at consecutive positions, all in [0, kv_len), runs
// from its first row's position; any other group computes its rows one at a
// time with the per-row gather, as band_fwd_kernel does.
//
// Non-finite K / V: as in band_fwd_kernel, a group whose output met a
// non-finite value (V rows of keys outside a row's window meet p = 0, and
// 0 * Inf = NaN) runs again with the staged V operands sanitised, and each
// row's own non-finite V values are put back from its entries.
#include "esa_band.hpp"
#include "esa_gather.hpp"

namespace esa {

namespace {

template <int D, int G, Elem E, bool POS>
__global__ __launch_bounds__(64, 2) void window_fwd_kernel(BandArgs A) {
  using C = BandCfg<D>;
  using M = MmaT<E>;
  using V8 = typename M::v8;
  __shared__ __attribute__((aligned(1024))) uint16_t ks0[C::SLOT];
  __shared__ __attribute__((aligned(1024))) uint16_t ks1[C::SLOT];
  __shared__ __attribute__((aligned(1024))) uint16_t vs0[C::SLOT];
  __shared__ __attribute__((aligned(1024))) uint16_t vs1[C::SLOT];
  uint16_t* const slot[4] = {ks0, ks1, vs0, vs1};

  // ---- group of 16 G rows: XCD x takes the contiguous range [x per, (x + 1) per)
  const int bid = blockIdx.x;
  const int g = (bid & 7) * A.per_xcd + (bid >> 3);
  if (g >= A.n_groups) return;
  const int bh = g / A.ng, gq = g % A.ng;
  const int h = bh % A.H, b = bh / A.H;
  const int kvh = h / A.groups;

  const int lane = threadIdx.x;
  const int n = lane & 15, q = lane >> 4;
  const int r0 = gq * 16 * G;  // the group's first row (of q, o and lse)
  const int w = A.pc.w;
  const int n_rows = min(16 * G, A.q_len - r0);
  int base = r0;  // the first row's position
  if constexpr (POS) {
    int64_t p0 = A.positions[r0];
    p0 = p0 < 0 ? p0 + A.kv_len : p0;
    base = __builtin_amdgcn_readfirstlane((int)(p0 >= 0 && p0 < A.kv_len ? p0 : 0));
    bool bad = !(p0 >= 0 && p0 < A.kv_len);
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int r = r0 + 16 * u + n;
      if (r < A.q_len) {
        int64_t p = A.positions[r];
        p = p < 0 ? p + A.kv_len : p;
        bad |= !(p >= 0 && p < A.kv_len && p == (int64_t)base + 16 * u + n);
      }
    }
    if (wave_any(bad)) {
      // positions not consecutive (or out of range): the rows one at a time,
      // by the per-row gather, with the first K slot as its 384-float scratch
      GatherArgs Gr{};
      Gr.q = A.q; Gr.k = A.k; Gr.v = A.v; Gr.o = A.o; Gr.lse = A.lse;
      Gr.qsb = A.qsb; Gr.qsh = A.qsh; Gr.qss = A.qss;
      Gr.ksb = A.ksb; Gr.ksh = A.ksh; Gr.kss = A.kss;
      Gr.vsb = A.vsb; Gr.vsh = A.vsh; Gr.vss = A.vss;
      Gr.osb = A.osb; Gr.osh = A.osh; Gr.oss = A.oss;
      Gr.lsb = A.lsb; Gr.lsh = A.lsh;
      Gr.H = A.H; Gr.groups = A.groups; Gr.q_len = A.q_len; Gr.kv_len = A.kv_len; Gr.D = D;
      Gr.sm_scale = A.sm_scale;
      Gr.elem = A.elem;
      Gr.src.w = A.pc.w; Gr.src.kv_len = A.kv_len; Gr.src.pc = A.pc;
      Gr.src.positions = A.positions;
      for (int rr = 0; rr < n_rows; ++rr)
        gather_one_row_any<E, true>(Gr, b, h, r0 + rr, (float*)ks0, lane);
      return;
    }
  }
  // the group's keys [k0, k1): the windows of its rows (positions base ..
  // base + n_rows - 1)
  const int k0 = max(base - w + 1, 0);
  const int k1 = base + n_rows;
  const int n_pairs = (k1 - k0 + 31) / 32;
  // pair order: the group at position base starts at pair (-base / 16 G) mod
  // n_pairs and wraps around.  The next group's keys start 16 G keys later,
  // so its pair p is this group's pair p + 1: with this order the n_pairs
  // groups that share a pair all load it at the same step, while it is in L2
  const int pstart = (n_pairs - (base / (16 * G)) % n_pairs) % n_pairs;
  // row 16 u + n of the group: its window as offsets from k0
  int lo[G], hi[G];
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const int i = base + 16 * u + n;
    const bool ok = 16 * u + n < n_rows;
    lo[u] = ok ? max(i - w + 1, 0) - k0 : 1;
    hi[u] = ok ? i - k0 : 0;
  }

  {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int c = 0; c < C::SLOT / 512; ++c) *(u32x4*)(slot[s] + (c * 64 + lane) * 8) = z;
  }

  // ---- Q as the B operand: row 16 u + n, dims 32 s + 8 q .. + 8 for k-step s
  V8 qop[G][C::NS];
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const int r = r0 + 16 * u + n;
    const uint16_t* qrow = A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)r * A.qss;
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (r < A.q_len) raw = *(const u32x4*)(qrow + 32 * s + 8 * q);
      qop[u][s] = __builtin_bit_cast(V8, raw);
    }
  }

  const char* const kbase = (const char*)(A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh);
  const char* const vbase = (const char*)(A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh);
  const int kss2 = (int)A.kss * 2, vss2 = (int)A.vss * 2;
  lds_u16* const lk0 = (lds_u16*)ks0;
  lds_u16* const lk1 = (lds_u16*)ks1;
  lds_u16* const lv0 = (lds_u16*)vs0;
  lds_u16* const lv1 = (lds_u16*)vs1;
  int kofs[C::VLOADS], vofs[C::VLOADS];
#pragma unroll
  for (int t = 0; t < C::VLOADS; ++t) {
    const int R = (64 * t + lane) / C::CPR, pc = lane % C::CPR;
    kofs[t] = R * kss2 + 16 * kswz<D>(R, pc);
    vofs[t] = R * vss2 + 16 * vswz<D>(R, pc);
  }
  // chunk c (keys k0 + 16 c ..) -> slot dst: only the DMAs that reach one of
  // the group's keys; slot rows past them keep older contents (K: scores
  // no row keeps; V: rows that meet p = 0)
  constexpr int RPI = 64 / C::CPR;
  auto load_chunk = [&](const char* base, int ss2, const int* ofs, int c, lds_u16* dst) {
    const int c0 = k0 + 16 * c;
    const int rows = __builtin_amdgcn_readfirstlane(max(min(k1 - c0, 16), 0));
    const int nl = (rows + RPI - 1) / RPI;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(base + (int64_t)min(c0, k1) * ss2), (short)0, rows * ss2, 0x00020000);
#pragma unroll
    for (int t = 0; t < C::VLOADS; ++t) {
      if (t < nl)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + 512 * t), 16, ofs[t], 0,
                                                 0, 0);
    }
  };

  int krd[C::NS];
#pragma unroll
  for (int s = 0; s < C::NS; ++s) krd[s] = n * C::ROWB + 16 * kswz<D>(n, 4 * s + q);
  int vrd[C::NV];
#pragma unroll
  for (int s = 0; s < C::NV; ++s) {
    const int R = 4 * q + (n >> 2);
    const int dim0 = C::CW * (n & 3) + 4 * s;
    vrd[s] = R * C::ROWB + 16 * vswz<D>(R, dim0 >> 3) + 2 * (dim0 & 7);
  }

  const float scale = A.scale_log2;
  float m_run[G], l_run[G], n_run[G];
  f32x4 oacc[G][C::NV];

  auto scores = [&](const V8 (&kb)[C::NS], const V8 (&qb)[C::NS]) {
    f32x4 sacc = M::mfma16(kb[0], qb[0], f32x4{});
#pragma unroll
    for (int s = 1; s < C::NS; ++s) sacc = M::mfma16(kb[s], qb[s], sacc);
    return sacc;
  };

  auto run = [&](auto san) {
#pragma unroll
    for (int u = 0; u < G; ++u) {
      m_run[u] = -INFINITY;
      l_run[u] = 0.f;
      n_run[u] = 0.f;
#pragma unroll
      for (int s = 0; s < C::NV; ++s) oacc[u][s] = f32x4{};
    }
    {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slot zeros are in LDS
      load_chunk(kbase, kss2, kofs, 2 * pstart, lk0);
      load_chunk(kbase, kss2, kofs, 2 * pstart + 1, lk1);
      load_chunk(vbase, vss2, vofs, 2 * pstart, lv0);
      load_chunk(vbase, vss2, vofs, 2 * pstart + 1, lv1);
    }
    for (int st = 0, p = pstart; st < n_pairs; ++st, p = p + 1 == n_pairs ? 0 : p + 1) {
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // this pair's K and V are in LDS
      V8 ka[C::NS], kb[C::NS];
      s16x4 ta[C::NV], tb[C::NV];
#pragma unroll
      for (int s = 0; s < C::NS; ++s) {
        ka[s] = *(const V8*)((const char*)ks0 + krd[s]);
        kb[s] = *(const V8*)((const char*)ks1 + krd[s]);
      }
#pragma unroll
      for (int s = 0; s < C::NV; ++s) {
        ta[s] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((const char*)vs0 + vrd[s]));
        tb[s] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((const char*)vs1 + vrd[s]));
      }
      if constexpr (decltype(san)::value) {
#pragma unroll
        for (int s = 0; s < C::NV; ++s) {
          u32x2 x = __builtin_bit_cast(u32x2, ta[s]), y = __builtin_bit_cast(u32x2, tb[s]);
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            x[e] = sanitize2<E>(x[e]);
            y[e] = sanitize2<E>(y[e]);
          }
          ta[s] = __builtin_bit_cast(s16x4, x);
          tb[s] = __builtin_bit_cast(s16x4, y);
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // slots read: refill them
      if (st + 1 < n_pairs) {
        const int pn = p + 1 == n_pairs ? 0 : p + 1;
        load_chunk(kbase, kss2, kofs, 2 * pn, lk0);
        load_chunk(kbase, kss2, kofs, 2 * pn + 1, lk1);
        load_chunk(vbase, vss2, vofs, 2 * pn, lv0);
        load_chunk(vbase, vss2, vofs, 2 * pn + 1, lv1);
      }
      // this lane's keys: 32 p + 4 q + e (chunk a) and 32 p + 16 + 4 q + e
      // (chunk b), as offsets from k0
      const int ka0 = 32 * p + 4 * q, kb0 = ka0 + 16;
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const f32x4 sa = scores(ka, qop[u]);
        const f32x4 sb = scores(kb, qop[u]);
        // scores outside the row's window: -inf
        float x[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[e] = (ka0 + e >= lo[u] && ka0 + e <= hi[u]) ? sa[e] * scale : -INFINITY;
          x[4 + e] = (kb0 + e >= lo[u] && kb0 + e <= hi[u]) ? sb[e] * scale : -INFINITY;
        }
        float xm = max_nq(max_nq(max_nq(x[0], x[1]), max_nq(x[2], x[3])),
                          max_nq(max_nq(x[4], x[5]), max_nq(x[6], x[7])));
        xm = row4_max(xm);
        const float m_use = m_run[u] == -INFINITY ? 0.f : m_run[u];
        const float rm = xm - m_use;
        const float thr = m_run[u] == -INFINITY ? -INFINITY : kRescaleSlack;
        const bool grow = rm > thr;
        float delta = 0.f;
        if (wave_any(grow)) {
          delta = grow ? rm : 0.f;
          const float alpha = grow ? __builtin_amdgcn_exp2f(m_run[u] - (m_use + delta)) : 1.0f;
          l_run[u] *= alpha;
          n_run[u] *= alpha;
#pragma unroll
          for (int v = 0; v < C::NV; ++v) oacc[u][v] *= alpha;
          m_run[u] = grow ? m_use + delta : m_run[u];
        }
        const float off = m_use + delta;
        uint32_t pw[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float p0 = __builtin_amdgcn_exp2f(x[2 * c] - off);
          const float p1 = __builtin_amdgcn_exp2f(x[2 * c + 1] - off);
          l_run[u] += p0;
          l_run[u] += p1;
          const uint32_t b0 = (uint32_t)M::bits(p0), b1 = (uint32_t)M::bits(p1);
          // O is normalised by the probabilities PV used (rounded to the input type)
          n_run[u] += M::val(b0);
          n_run[u] += M::val(b1);
          pw[c] = b0 | (b1 << 16);
        }
        const u32x4 pq = {pw[0], pw[1], pw[2], pw[3]};
        const V8 pop = __builtin_bit_cast(V8, pq);
#pragma unroll
        for (int s = 0; s < C::NV; ++s) {
          const s16x4 vv[2] = {ta[s], tb[s]};
          oacc[u][s] = M::mfma16(__builtin_bit_cast(V8, vv), pop, oacc[u][s]);
        }
      }
    }
  };

  run(std::integral_constant<bool, false>{});
  bool bad = false;
#pragma unroll
  for (int u = 0; u < G; ++u) bad |= !sum_finite(oacc[u]);
  const bool rerun = wave_any(bad);
  if (rerun) run(std::integral_constant<bool, true>{});

  // ---- epilogue: lane (n, q) holds O^T[dim][row n] for dims CW q .. CW q + CW;
  // a row's sums are split over its 4 lanes (each summed its own keys)
#pragma unroll
  for (int u = 0; u < G; ++u) {
    float l_tot = l_run[u], n_tot = n_run[u];
    l_tot += __shfl_xor(l_tot, 16, 64);
    l_tot += __shfl_xor(l_tot, 32, 64);
    n_tot += __shfl_xor(n_tot, 16, 64);
    n_tot += __shfl_xor(n_tot, 32, 64);
    const int r = r0 + 16 * u + n, i = base + 16 * u + n;  // row, position
    if (r >= A.q_len) continue;
    const float inv = n_tot > 0.f ? 1.f / n_tot : 0.f;
    uint16_t* orow = A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)r * A.oss;
#pragma unroll
    for (int t = 0; t < C::NV / 2; ++t) {
      V8 ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ov[e] = (typename M::s)(oacc[u][2 * t][e] * inv);
        ov[4 + e] = (typename M::s)(oacc[u][2 * t + 1][e] * inv);
      }
      *(V8*)(orow + C::CW * q + 8 * t) = ov;
    }
    if (A.lse && q == 0) {
      const float lse = l_tot > 0.f ? (m_run[u] + __log2f(l_tot)) * 0.69314718055994530942f
                                    : -INFINITY;
      A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + r] = lse;
    }
    if (rerun) {
      int dim0[C::CW / 4];
#pragma unroll
      for (int gg = 0; gg < C::CW / 4; ++gg) dim0[gg] = C::CW * q + 4 * gg;
      uint64_t pos, neg, nan;
      nonfinite_v<E>(A.pc, h, i, A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh, A.vss, dim0,
                     pos, neg, nan);
      for (uint64_t any = pos | neg | nan; any != 0ull; any &= any - 1ull) {
        const int bit = __builtin_ctzll(any);
        orow[C::CW * q + bit] = nonfinite_value<E>(pos, neg, nan, bit);
      }
    }
  }
}

}  // namespace

bool window_fwd_applies(const BandArgs& a, int head_dim) {
  return a.pc.a == 0.0f && a.d_real == head_dim && (head_dim == 64 || head_dim == 128);
}

// rows per wave: 16 WINDOW_G (two 16-row groups share each chunk's staging)
constexpr int WINDOW_G = 2;

template <int D, Elem E>
void launch_window_d(const BandArgs& a, hipStream_t stream) {
  BandArgs w = a;
  w.ng = (a.q_len + 16 * WINDOW_G - 1) / (16 * WINDOW_G);
  const int64_t n = (int64_t)a.n_groups / a.ng * w.ng;  // batch * H * ng
  w.n_groups = (int)n;
  w.per_xcd = (int)((n + 7) / 8);
  const dim3 grid((unsigned)(8 * w.per_xcd));
  if (a.positions)
    window_fwd_kernel<D, WINDOW_G, E, true><<<grid, 64, 0, stream>>>(w);
  else
    window_fwd_kernel<D, WINDOW_G, E, false><<<grid, 64, 0, stream>>>(w);
}

hipError_t launch_window_fwd(const BandArgs& a, int head_dim, hipStream_t stream) {
  if (a.n_groups <= 0) return hipSuccess;
  if (a.elem == (int)Elem::f16) {
    if (head_dim == 128)
      launch_window_d<128, Elem::f16>(a, stream);
    else
      launch_window_d<64, Elem::f16>(a, stream);
  } else {
    if (head_dim == 128)
      launch_window_d<128, Elem::bf16>(a, stream);
    else
      launch_window_d<64, Elem::bf16>(a, stream);
  }
  return hipGetLastError();
}

}  // namespace esa
