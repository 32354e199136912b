// Band-gathered dQ and dK / dV of the elastic prefill backward (gfx950).
//
// band_dq_kernel replaces the dQ half of the reference's Triton backward
// (elastic_sparse_attention.py:168-233) the way band_fwd_kernel replaces the
// forward: one wave per 16 query rows (a group); for each entry j of the
// rows' index lists (a band) the keys [lo_j, lo_j + 16) are staged in LDS
// (K and V rows by buffer_load ... lds), and per band pair
//
//   S^T  = K Q^T      D/32 x v_mfma_f32_16x16x32_bf16 (A = K rows from LDS,
//                     B = Q in registers)
//   dP^T = V dO^T     D/32 MFMAs (A = V rows from LDS, B = dO in registers)
//   pick             the lane holding the row's key of the band takes its
//                     score and dP: P = exp2(S scale log2e - lse2) (exact:
//                     the forward's log-sum-exp), dS = P (dP - delta)
//   dQ^T += K^T dS^T  D/16 MFMAs over the two bands' 32 keys (A = K^T read
//                     with ds_read_b64_tr_b16 from the same K slot, B = dS
//                     as bf16 at the key's register slot)
//
// dQ = scale * dQ^T^T.  Each row's key of a band is selected in exactly one
// chunk (bands wider than 16 keys get a tail pass), so every valid (row,
// key) pair contributes once, as in :191-228.  band_dkdv_kernel (below) is
// the key-major counterpart for dK and dV; dkdv_kernel (esa_bwd.hip) is the
// block-sparse one.  At interpolation weight 0 (a sliding window) dQ runs
// window_dq_kernel (32-row groups over the window keys in 16-key chunks) and
// dK / dV band_dkdv_kernel's WIN form (the block's window rows in 32-row
// steps), in place of 64 bands.  Operand layouts: esa_band.hpp.
#include "esa_band.hpp"

namespace esa {

// VSKIP: issue only the K and V DMAs that reach a band row (see
// load_rows); the host picks it where many bands are narrower than 16 keys,
// as for the forward's K DMA skip.
// PREP: the kernel forms its rows' delta = rowsum(dO * O) and lse2 = lse *
// log2(e) itself (instead of reading them) and stores both for the band
// dK/dV kernel, which then runs after it; block 0 also clears the split
// arrival counters.  Used when both halves are band kernels, so no separate
// pass re-reads O and dO.
template <int D, bool VSKIP, bool PREP, Elem E>
__global__ __launch_bounds__(64, 2) void band_dq_kernel(BwdArgs A, const float* lse2) {
  using M = MmaT<E>;
  using V8 = typename M::v8;
  using C = BandCfg<D>;
  if (PREP && A.split_parts > 1 && blockIdx.x == 0)
    for (int t = threadIdx.x; t < A.n_bkv * A.split_blocks; t += 64) A.part_cnt[t] = 0;
  __shared__ __attribute__((aligned(1024))) uint16_t ks0[C::SLOT];
  __shared__ __attribute__((aligned(1024))) uint16_t ks1[C::SLOT];
  __shared__ __attribute__((aligned(1024))) uint16_t vs0[C::SLOT];
  __shared__ __attribute__((aligned(1024))) uint16_t vs1[C::SLOT];
  uint16_t* const slot[4] = {ks0, ks1, vs0, vs1};

  // ---- group: XCD x takes the contiguous range [x per, (x + 1) per)
  const int bid = blockIdx.x;
  const int g = (bid & 7) * A.per_xcd + (bid >> 3);
  if (g >= A.n_groups) return;
  const int bh = g / A.ng, gq = g % A.ng;
  const int h = bh % A.H, b = bh / A.H;
  const int kvh = h / A.groups;

  const int lane = threadIdx.x;
  const int n = lane & 15, q = lane >> 4;
  const int i = gq * 16 + n;
  const bool row_ok = i < A.q_len;

  {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int c = 0; c < C::SLOT / 512; ++c) *(u32x4*)(slot[s] + (c * 64 + lane) * 8) = z;
  }

  // Q and dO of this lane's row as B operands: dims 32 s + 8 q .. + 8
  V8 qop[C::NS], dop[C::NS];
  {
    const uint16_t* qr = A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)i * A.qss;
    const uint16_t* dr =
        A.dout + (int64_t)b * A.dosb + (int64_t)h * A.dosh + (int64_t)i * A.doss;
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
      u32x4 qraw = {0u, 0u, 0u, 0u}, draw = {0u, 0u, 0u, 0u};
      if (row_ok) {
        qraw = *(const u32x4*)(qr + 32 * s + 8 * q);
        draw = *(const u32x4*)(dr + 32 * s + 8 * q);
      }
      qop[s] = __builtin_bit_cast(V8, qraw);
      dop[s] = __builtin_bit_cast(V8, draw);
    }
  }
  float l2 = 0.f, dl = 0.f;
  if constexpr (PREP) {
    // rowsum(dO * O) in prep_kernel's order, so both give the same bits:
    // there, lane g of 16 sums dims D/16 g .. + D/16 in sequence and the 16
    // sums meet in an xor butterfly (strides 8, 4, 2, 1).  Here lane (n, q)
    // holds dims 32 s + 8 q .. + 8; each product of two bf16 values is exact
    // in float32, so only the order of the additions matters.
    float hs[C::NS][2];  // sequential sums of each D/16-dim piece
    {
      u32x4 raw[C::NS];
      const uint16_t* orow =
          A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)i * A.oss;
#pragma unroll
      for (int s = 0; s < C::NS; ++s) {
        raw[s] = u32x4{0u, 0u, 0u, 0u};
        if (row_ok) raw[s] = *(const u32x4*)(orow + 32 * s + 8 * q);
      }
      constexpr int PER = D / 16;
#pragma unroll
      for (int s = 0; s < C::NS; ++s)
#pragma unroll
        for (int k = 0; k < 8 / PER; ++k) {
          float acc = 0.f;
#pragma unroll
          for (int e = PER * k; e < PER * k + PER; ++e) {
            const uint32_t w = raw[s][e / 2];
            const float ov = M::val((e & 1) ? (w >> 16) : (w & 0xffffu));
            acc += ov * (float)dop[s][e];
          }
          hs[s][k] = acc;
        }
    }
    if constexpr (D == 128) {
      // piece 4 s + q: strides 8 and 4 stay in the lane (s ^ 2, s ^ 1),
      // 2 and 1 cross to lanes ^ 32 and ^ 16
      float t = (hs[0][0] + hs[2][0]) + (hs[1][0] + hs[3][0]);
      t += __shfl_xor(t, 32, 64);
      t += __shfl_xor(t, 16, 64);
      dl = t;
    } else {
      // piece 8 s + 2 q + k: stride 8 is s ^ 1, 4 and 2 cross to lanes ^ 32
      // and ^ 16, 1 is k ^ 1
      float t0 = hs[0][0] + hs[1][0], t1 = hs[0][1] + hs[1][1];
      t0 += __shfl_xor(t0, 32, 64);
      t1 += __shfl_xor(t1, 32, 64);
      t0 += __shfl_xor(t0, 16, 64);
      t1 += __shfl_xor(t1, 16, 64);
      dl = t0 + t1;
    }
    if (row_ok) {
      // kept finite: masked scores enter as -inf, and -inf - (-inf) would be NaN
      l2 = fmaxf(A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + i] * 1.4426950408889634f,
                 -3.0e38f);
      if (q == 0) {
        const int64_t at = ((int64_t)b * A.H + h) * A.qpad + i;
        A.delta[at] = dl;
        A.delta[(int64_t)A.B * A.H * A.qpad + at] = l2;  // the lse2 half of the workspace
      }
    }
  } else {
    if (row_ok) {
      const int64_t at = ((int64_t)b * A.H + h) * A.qpad + i;
      l2 = lse2[at];
      dl = A.delta[at];
    }
  }

  uint32_t kd[4];  // the row's key offsets (band_rows)
  int info1;       // slot (q, r)'s descriptor in lane 16 q + r
  // entry rotation, A.rot_dq 64ths of an entry per group dispatched on the
  // XCD (launch_band_dq picks the rate)
  // (unsigned: the product wraps for grids near 2^31 blocks; only the value
  // mod 64 matters)
  band_rows(A.pc, h, i, row_ok, q, n,
              (int)(((unsigned)(bid >> 3) * (unsigned)A.rot_dq / 64u) & 63u), kd, info1);

  const char* const kbase = (const char*)(A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh);
  const char* const vbase = (const char*)(A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh);
  const int kss2 = (int)A.kss * 2, vss2 = (int)A.vss * 2;
  lds_u16* const lk0 = (lds_u16*)ks0;
  lds_u16* const lk1 = (lds_u16*)ks1;
  lds_u16* const lv0 = (lds_u16*)vs0;
  lds_u16* const lv1 = (lds_u16*)vs1;
  // DMA t, lane l fills slot row R = (64 t + l) / CPR, physical chunk l % CPR
  // (both matrices use the K swizzle: read as 16-row operands, K also
  // transposed): byte offsets from the band's first row
  int kofs[C::VLOADS], vofs[C::VLOADS];
#pragma unroll
  for (int t = 0; t < C::VLOADS; ++t) {
    const int R = (64 * t + lane) / C::CPR, pc = lane % C::CPR;
    kofs[t] = R * kss2 + 16 * kswz<D>(R, pc);
    vofs[t] = R * vss2 + 16 * kswz<D>(R, pc);
  }
  // K or V rows of band `bi` -> slot dst, through a buffer resource over the
  // band's W rows (rows past the band read as zeros without a fetch).  Each
  // takes VLOADS DMAs, or with VSKIP only the ceil(W / RPI) that reach a
  // band row: slot rows past them then keep older contents.  Old V rows only
  // feed dP of keys no row picks; old K rows meet dS = 0 in dQ^T += K^T dS^T
  // (0 * Inf = NaN for a non-finite one flags the group, and bwd_fix_kernel
  // recomputes it).  The vmcnt waits count the DMAs issued.
  constexpr int RPI = 64 / C::CPR;  // slot rows per DMA
  auto n_loads = [&](int bi) { return (min((int)((uint32_t)bi >> 24), 16) + RPI - 1) / RPI; };
  auto load_rows = [&](const char* base, int ss2, const int* ofs, int bi, lds_u16* dst,
                       bool all) {
    const int lo = bi & 0xffffff, wdt = (int)((uint32_t)bi >> 24);
    const int nl = __builtin_amdgcn_readfirstlane(n_loads(bi));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(base + (int64_t)lo * ss2), (short)0,
        __builtin_amdgcn_readfirstlane(min(wdt, 16) * ss2), 0x00020000);
#pragma unroll
    for (int t = 0; t < C::VLOADS; ++t) {
      if (all || t < nl)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + 512 * t), 16, ofs[t], 0,
                                                 0, 0);
    }
  };
  auto load_k = [&](int bi, lds_u16* dst) { load_rows(kbase, kss2, kofs, bi, dst, !VSKIP); };
  auto load_v = [&](int bi, lds_u16* dst) { load_rows(vbase, vss2, vofs, bi, dst, !VSKIP); };
  // s_waitcnt vmcnt(n) for a count known only at run time (0 .. 8)
  auto wait_vm = [&](int n) {
    switch (n) {
      case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
      case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
      case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
      case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
      case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
      case 5: __builtin_amdgcn_s_waitcnt(0x0F75); break;
      case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
      case 7: __builtin_amdgcn_s_waitcnt(0x0F77); break;
      default: __builtin_amdgcn_s_waitcnt(0x0F78); break;
    }
  };
  static_assert(2 * C::VLOADS <= 8, "wait_vm covers at most 8 DMAs in flight");

  // row operand reads: lane (m = n, q) reads slot row n, dims 32 s + 8 q .. + 8
  int rrd[C::NS];
#pragma unroll
  for (int s = 0; s < C::NS; ++s) rrd[s] = n * C::ROWB + 16 * kswz<D>(n, 4 * s + q);
  // transposed reads (K^T operand of dQ^T) for slice s: lane x of its 16-lane
  // group reads slot row 4 q + x/4, dims CW (x%4) + 4 s .. + 3
  int trd[C::NV];
#pragma unroll
  for (int s = 0; s < C::NV; ++s) {
    const int R = 4 * q + (n >> 2), dim0 = C::CW * (n & 3) + 4 * s;
    trd[s] = R * C::ROWB + 16 * kswz<D>(R, dim0 >> 3) + 2 * (dim0 & 7);
  }
  auto read_rows = [&](const uint16_t* src, V8 (&op)[C::NS]) {
#pragma unroll
    for (int s = 0; s < C::NS; ++s) op[s] = *(const V8*)((const char*)src + rrd[s]);
  };
  auto read_tr = [&](const uint16_t* src, s16x4 (&op)[C::NV]) {
#pragma unroll
    for (int s = 0; s < C::NV; ++s)
      op[s] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((const char*)src + trd[s]));
  };
  auto product = [&](const V8 (&a)[C::NS], const V8 (&bop)[C::NS]) {
    f32x4 acc = M::mfma16(a[0], bop[0], f32x4{});
#pragma unroll
    for (int s = 1; s < C::NS; ++s) acc = M::mfma16(a[s], bop[s], acc);
    return acc;
  };

  const float scale2 = A.scale_log2;
  // dS of this row's key in chunk [c0, c0 + 16) of a band, as bf16 at the
  // key's register slot of the lane holding it (0 elsewhere)
  // d = the row's key minus the chunk's first key (no key in the chunk: d <
  // 0 or d >= 16); this lane holds the key when d >> 2 == q (an arithmetic
  // shift keeping d < 0 out)
  auto ds_word = [&](const f32x4& sacc, const f32x4& pacc, int d) -> uint64_t {
    const bool has = (d >> 2) == q;
    const int e = d & 3;
    const float s01 = (e & 1) ? sacc[1] : sacc[0];
    const float s23 = (e & 1) ? sacc[3] : sacc[2];
    const float dp01 = (e & 1) ? pacc[1] : pacc[0];
    const float dp23 = (e & 1) ? pacc[3] : pacc[2];
    const float s = (e & 2) ? s23 : s01;
    const float dp = (e & 2) ? dp23 : dp01;
    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s, scale2, -l2));
    const uint32_t w = (uint32_t)M::bits(p * (dp - dl));
    return has ? ((uint64_t)w << (16 * e)) : 0ull;
  };

  f32x4 dqacc[C::NV];
#pragma unroll
  for (int s = 0; s < C::NV; ++s) dqacc[s] = f32x4{};
  // dQ^T += K^T dS^T over two bands' keys
  auto dq_step = [&](const s16x4 (&ta)[C::NV], const s16x4 (&tb)[C::NV], uint64_t wa,
                     uint64_t wb) {
    const u32x4 sq = {(uint32_t)wa, (uint32_t)(wa >> 32), (uint32_t)wb, (uint32_t)(wb >> 32)};
    const V8 sop = __builtin_bit_cast(V8, sq);
#pragma unroll
    for (int s = 0; s < C::NV; ++s) {
      const s16x4 kk[2] = {ta[s], tb[s]};
      dqacc[s] = M::mfma16(__builtin_bit_cast(V8, kk), sop, dqacc[s]);
    }
  };

  // ---- band pairs: per pair, K reads, then K of the next pair; V reads,
  // then V of the next pair.  So before the V wait exactly the next pair's K
  // DMAs may be newer, and before the K wait this pair's V DMAs (2 VLOADS of
  // each, or with VSKIP as many as load_k / load_v issued).
  constexpr int kWaitPair = (0xF70 & ~0xF) | ((2 * C::VLOADS) & 0xF) |
                            (((2 * C::VLOADS) >> 4) << 14);  // vmcnt(2 VLOADS)
  constexpr int kWaitLds = 0xC07F;                           // lgkmcnt(0)
  const int lane_key = 4 * n;
  {
    const int i0 = __builtin_amdgcn_readlane(info1, 0);
    const int i1 = __builtin_amdgcn_readlane(info1, 1);
    __builtin_amdgcn_s_waitcnt(kWaitLds);  // the slot zeros are in LDS
    load_k(i0, lk0);
    load_k(i1, lk1);
    load_v(i0, lv0);
    load_v(i1, lv1);
  }
  for (int qj = 0; qj < 4; ++qj) {
    const bool more = qj < 3;
#pragma unroll
    for (int rp = 0; rp < 8; ++rp) {
      const int ra = 2 * rp, rb = 2 * rp + 1;
      const int ia = __builtin_amdgcn_readlane(info1, 16 * qj + ra);
      const int ib = __builtin_amdgcn_readlane(info1, 16 * qj + rb);
      // next pair's (at rp = 7 slots 0 and 1 of lane group qj + 1)
      int na = 0, nb = 0;
      if (rp < 7 || more) {
        na = __builtin_amdgcn_readlane(info1, 16 * qj + ra + 2);
        nb = __builtin_amdgcn_readlane(info1, 16 * qj + rb + 2);
      }
      const bool live = (ia | ib) != 0;
      // this pair's K is in LDS
      if constexpr (VSKIP)
        wait_vm(n_loads(ia) + n_loads(ib));
      else
        __builtin_amdgcn_s_waitcnt(kWaitPair);
      f32x4 sa, sb;
      s16x4 ta[C::NV], tb[C::NV];
      if (live) {
        {
          V8 ka[C::NS], kb[C::NS];
          read_rows(ks0, ka);
          read_rows(ks1, kb);
          sa = product(ka, qop);
          sb = product(kb, qop);
        }
        __builtin_amdgcn_sched_barrier(0);
        read_tr(ks0, ta);
        read_tr(ks1, tb);
      }
      __builtin_amdgcn_s_waitcnt(kWaitLds);  // K slots read: refill them
      load_k(na, lk0);
      load_k(nb, lk1);
      // this pair's V is in LDS
      if constexpr (VSKIP)
        wait_vm(n_loads(na) + n_loads(nb));
      else
        __builtin_amdgcn_s_waitcnt(kWaitPair);
      V8 va[C::NS], vb[C::NS];
      if (live) {
        read_rows(vs0, va);
        read_rows(vs1, vb);
      }
      __builtin_amdgcn_s_waitcnt(kWaitLds);  // V slots read: refill them
      load_v(na, lv0);
      load_v(nb, lv1);
      if (live) {
        const f32x4 pa = product(va, dop);
        const f32x4 pb = product(vb, dop);
        // both bands' key offsets: bytes ra % 4, rb % 4 of word rp / 2
        const uint32_t dw =
            (uint32_t)__builtin_amdgcn_ds_bpermute(lane_key + 64 * qj, (int)kd[rp >> 1]);
        const uint64_t wa = ds_word(sa, pa, (int)((dw >> (16 * (rp & 1))) & 0xFFu));
        const uint64_t wb = ds_word(sb, pb, (int)((dw >> (16 * (rp & 1) + 8)) & 0xFFu));
        dq_step(ta, tb, wa, wb);
      }
    }
  }

  // ---- tail: keys of bands wider than 16, one 16-key chunk at a time (the
  // pair's second half is ks1 with dS = 0)
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  const bool wide = wave_any(((uint32_t)info1 >> 24) > 16u);  // some slot's band
  for (int j = 0; j < 64 && wide; ++j) {
    const int qj = j >> 4, r = j & 15;
    const int bi = __builtin_amdgcn_readlane(info1, j);  // slot (qj, r)
    // (the words as opaque values first: selects between loads of kd would
    // become a load at a selected address, which puts kd in scratch)
    uint32_t k0 = kd[0], k1 = kd[1], k2 = kd[2], k3 = kd[3];
    asm volatile("" : "+v"(k0), "+v"(k1), "+v"(k2), "+v"(k3));
    const uint32_t w4 = (r & 8) ? ((r & 4) ? k3 : k2) : ((r & 4) ? k1 : k0);
    const uint32_t dw = (uint32_t)__builtin_amdgcn_ds_bpermute(lane_key + 64 * qj, (int)w4);
    const int d = (int)((dw >> (8 * (r & 3))) & 0xFFu);  // 0xFF: no key
    const int lo = bi & 0xffffff, wdt = (int)((uint32_t)bi >> 24);
    for (int c0 = lo + 16; c0 < lo + wdt; c0 += 16) {
      const int ci = c0 | (min(lo + wdt - c0, 16) << 24);
      __builtin_amdgcn_s_waitcnt(kWaitLds);
      load_k(ci, lk0);
      load_v(ci, lv0);
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      V8 kt[C::NS], vt[C::NS];
      s16x4 tt[C::NV], tz[C::NV];
      read_rows(ks0, kt);
      read_rows(vs0, vt);
      read_tr(ks0, tt);
      read_tr(ks1, tz);
      const f32x4 st = product(kt, qop);
      const f32x4 pt = product(vt, dop);
      dq_step(tt, tz, ds_word(st, pt, d == 0xFF ? -1 : d - (c0 - lo)), 0ull);
    }
  }

  // ---- the group's non-finite flag (staged K rows a row does not list meet
  // dS = 0 in dQ^T, and 0 * Inf is NaN: bwd_fix_kernel recomputes such a
  // group exactly)
  {
    const bool bad = wave_any(!sum_finite(dqacc));
    if (lane == 0) A.flags[g] = bad ? 1 : 0;
  }
  // ---- dQ = scale * dQ^T^T: lane (n, q) holds dims CW q + 4 s + e of row n
  if (row_ok) {
    uint16_t* dqr = A.dq + (int64_t)b * A.dqsb + (int64_t)h * A.dqsh + (int64_t)i * A.dqss;
#pragma unroll
    for (int t = 0; t < C::NV / 2; ++t) {
      V8 ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ov[e] = (typename M::s)(dqacc[2 * t][e] * A.sm_scale);
        ov[4 + e] = (typename M::s)(dqacc[2 * t + 1][e] * A.sm_scale);
      }
      *(V8*)(dqr + C::CW * q + 8 * t) = ov;
    }
  }
}

// ---------------------------------------------------------------------------
// Window dQ over 32-row groups (interpolation weight 0, layer 0): one wave
// per (batch, head, 32-row group [r0, r0 + 32)), two 16-row halves u that
// share every staged pair.  The group's keys [max(r0 - w + 1, 0),
// min(r0 + 32, q_len)) go through the slots in 16-key chunks, two per pair
// (three pairs, 95 keys, at w = 64 for 32 rows, against three, 79 keys,
// for each 16-row group walked alone), so each row waits for half as many
// pairs for the same MFMAs.  Same box,
// layer-0 backward against 16-row groups: B=1 H=32 L=32768 0.805 -> 0.768
// ms, B=1 H=8 L=131072 -4%, B=8 H=16 L=4096 D=64 -5% (the pair order below
// 0.8-1.8% of that).  Per
// pair: S^T = K Q^T and dP^T = V dO^T for each half, dS at the keys of each
// row's window, dQ^T += K^T dS^T.  The group's pair p is the next group's
// pair p - 1, so each group starts at pair (-group) mod n_pairs and wraps
// around: the groups sharing a pair load it at the same step.  Each half
// writes the flag byte and delta / lse2 (PREP) of its 16-row group as
// band_dq_kernel does, so bwd_fix_kernel and the dK / dV kernel read the
// same workspace.
template <int D, bool PREP, Elem E>
__global__ __launch_bounds__(64, 2) void window_dq_kernel(BwdArgs A, const float* lse2) {
  using M = MmaT<E>;
  using V8 = typename M::v8;
  using C = BandCfg<D>;
  constexpr int G = 2;
  if (PREP && A.split_parts > 1 && blockIdx.x == 0)
    for (int t = threadIdx.x; t < A.n_bkv * A.split_blocks; t += 64) A.part_cnt[t] = 0;
  __shared__ __attribute__((aligned(1024))) uint16_t ks0[C::SLOT];
  __shared__ __attribute__((aligned(1024))) uint16_t ks1[C::SLOT];
  __shared__ __attribute__((aligned(1024))) uint16_t vs0[C::SLOT];
  __shared__ __attribute__((aligned(1024))) uint16_t vs1[C::SLOT];
  uint16_t* const slot[4] = {ks0, ks1, vs0, vs1};

  // ---- group: XCD x takes the contiguous range [x per, (x + 1) per)
  const int ng2 = (A.q_len + 16 * G - 1) / (16 * G);
  const int n2 = A.B * A.H * ng2;
  const int per2 = (n2 + 7) / 8;
  const int bid = blockIdx.x;
  const int g = (bid & 7) * per2 + (bid >> 3);
  if (g >= n2) return;
  const int bh = g / ng2, gq = g % ng2;
  const int h = bh % A.H, b = bh / A.H;
  const int kvh = h / A.groups;

  const int lane = threadIdx.x;
  const int n = lane & 15, q = lane >> 4;
  const int r0 = gq * 16 * G;

  {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int c = 0; c < C::SLOT / 512; ++c) *(u32x4*)(slot[s] + (c * 64 + lane) * 8) = z;
  }

  // Q and dO of row 16 u + n as B operands: dims 32 s + 8 q .. + 8
  V8 qop[G][C::NS], dop[G][C::NS];
  float l2[G], dl[G];
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const int i = r0 + 16 * u + n;
    const bool row_ok = i < A.q_len;
    const uint16_t* qr = A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)i * A.qss;
    const uint16_t* dr =
        A.dout + (int64_t)b * A.dosb + (int64_t)h * A.dosh + (int64_t)i * A.doss;
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
      u32x4 qraw = {0u, 0u, 0u, 0u}, draw = {0u, 0u, 0u, 0u};
      if (row_ok) {
        qraw = *(const u32x4*)(qr + 32 * s + 8 * q);
        draw = *(const u32x4*)(dr + 32 * s + 8 * q);
      }
      qop[u][s] = __builtin_bit_cast(V8, qraw);
      dop[u][s] = __builtin_bit_cast(V8, draw);
    }
    l2[u] = 0.f;
    dl[u] = 0.f;
    if constexpr (PREP) {
      // rowsum(dO * O) in prep_kernel's order (as band_dq_kernel forms it)
      float hs[C::NS][2];
      {
        u32x4 raw[C::NS];
        const uint16_t* orow =
            A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)i * A.oss;
#pragma unroll
        for (int s = 0; s < C::NS; ++s) {
          raw[s] = u32x4{0u, 0u, 0u, 0u};
          if (row_ok) raw[s] = *(const u32x4*)(orow + 32 * s + 8 * q);
        }
        constexpr int PER = D / 16;
#pragma unroll
        for (int s = 0; s < C::NS; ++s)
#pragma unroll
          for (int k = 0; k < 8 / PER; ++k) {
            float acc = 0.f;
#pragma unroll
            for (int e = PER * k; e < PER * k + PER; ++e) {
              const uint32_t w = raw[s][e / 2];
              const float ov = M::val((e & 1) ? (w >> 16) : (w & 0xffffu));
              acc += ov * (float)dop[u][s][e];
            }
            hs[s][k] = acc;
          }
      }
      if constexpr (D == 128) {
        float t = (hs[0][0] + hs[2][0]) + (hs[1][0] + hs[3][0]);
        t += __shfl_xor(t, 32, 64);
        t += __shfl_xor(t, 16, 64);
        dl[u] = t;
      } else {
        float t0 = hs[0][0] + hs[1][0], t1 = hs[0][1] + hs[1][1];
        t0 += __shfl_xor(t0, 32, 64);
        t1 += __shfl_xor(t1, 32, 64);
        t0 += __shfl_xor(t0, 16, 64);
        t1 += __shfl_xor(t1, 16, 64);
        dl[u] = t0 + t1;
      }
      if (row_ok) {
        // kept finite: masked scores enter as -inf, and -inf - (-inf) would be NaN
        l2[u] = fmaxf(A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + i] * 1.4426950408889634f,
                      -3.0e38f);
        if (q == 0) {
          const int64_t at = ((int64_t)b * A.H + h) * A.qpad + i;
          A.delta[at] = dl[u];
          A.delta[(int64_t)A.B * A.H * A.qpad + at] = l2[u];
        }
      }
    } else {
      if (row_ok) {
        const int64_t at = ((int64_t)b * A.H + h) * A.qpad + i;
        l2[u] = lse2[at];
        dl[u] = A.delta[at];
      }
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
    vofs[t] = R * vss2 + 16 * kswz<D>(R, pc);
  }
  const int w = A.pc.w;
  const int k0 = max(r0 - w + 1, 0), k1 = min(r0 + 16 * G, A.q_len);
  const int n_pairs = (k1 - k0 + 31) / 32;
  // chunk c (keys k0 + 16 c ..) -> slot dst: only the DMAs that reach one of
  // the group's keys (rows past k1 are not loaded; a slot's rows past them
  // keep older contents, which meet dS = 0)
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
  int rrd[C::NS];
#pragma unroll
  for (int s = 0; s < C::NS; ++s) rrd[s] = n * C::ROWB + 16 * kswz<D>(n, 4 * s + q);
  int trd[C::NV];
#pragma unroll
  for (int s = 0; s < C::NV; ++s) {
    const int R = 4 * q + (n >> 2), dim0 = C::CW * (n & 3) + 4 * s;
    trd[s] = R * C::ROWB + 16 * kswz<D>(R, dim0 >> 3) + 2 * (dim0 & 7);
  }
  auto read_rows = [&](const uint16_t* src, V8 (&op)[C::NS]) {
#pragma unroll
    for (int s = 0; s < C::NS; ++s) op[s] = *(const V8*)((const char*)src + rrd[s]);
  };
  auto read_tr = [&](const uint16_t* src, s16x4 (&op)[C::NV]) {
#pragma unroll
    for (int s = 0; s < C::NV; ++s)
      op[s] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((const char*)src + trd[s]));
  };
  auto product = [&](const V8 (&a)[C::NS], const V8 (&bop)[C::NS]) {
    f32x4 acc = M::mfma16(a[0], bop[0], f32x4{});
#pragma unroll
    for (int s = 1; s < C::NS; ++s) acc = M::mfma16(a[s], bop[s], acc);
    return acc;
  };
  const float scale2 = A.scale_log2;
  // row 16 u + n's window as offsets from k0 (none past q_len)
  int lo_k[G], hi_k[G];
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const int i = r0 + 16 * u + n;
    const bool ok = i < A.q_len;
    lo_k[u] = ok ? max(i - w + 1, 0) - k0 : 1;
    hi_k[u] = ok ? i - k0 : 0;
  }
  // dS of this lane's 4 keys kb0 .. kb0 + 3 (offsets from k0) for row
  // 16 u + n as 16-bit values at their register slots; 0 outside its window
  auto win_words = [&](int u, const f32x4& sacc, const f32x4& pacc, int kb0) -> uint64_t {
    uint64_t wv = 0ull;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool in = kb0 + e >= lo_k[u] && kb0 + e <= hi_k[u];
      const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[e], scale2, -l2[u]));
      const uint64_t bits = (uint64_t)(uint32_t)M::bits(p * (pacc[e] - dl[u]));
      wv |= in ? bits << (16 * e) : 0ull;
    }
    return wv;
  };
  f32x4 dqacc[G][C::NV];
#pragma unroll
  for (int u = 0; u < G; ++u)
#pragma unroll
    for (int s = 0; s < C::NV; ++s) dqacc[u][s] = f32x4{};

  const int pstart = (n_pairs - gq % n_pairs) % n_pairs;
  __builtin_amdgcn_s_waitcnt(0xC07F);  // the slot zeros are in LDS
  load_chunk(kbase, kss2, kofs, 2 * pstart, lk0);
  load_chunk(kbase, kss2, kofs, 2 * pstart + 1, lk1);
  load_chunk(vbase, vss2, vofs, 2 * pstart, lv0);
  load_chunk(vbase, vss2, vofs, 2 * pstart + 1, lv1);
  for (int st = 0, p = pstart; st < n_pairs; ++st, p = p + 1 == n_pairs ? 0 : p + 1) {
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // this pair's K and V are in LDS
    f32x4 sa[G], sb[G];
    s16x4 ta[C::NV], tb[C::NV];
    V8 va[C::NS], vb[C::NS];
    {
      V8 ka[C::NS], kb[C::NS];
      read_rows(ks0, ka);
      read_rows(ks1, kb);
#pragma unroll
      for (int u = 0; u < G; ++u) {
        sa[u] = product(ka, qop[u]);
        sb[u] = product(kb, qop[u]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    read_tr(ks0, ta);
    read_tr(ks1, tb);
    read_rows(vs0, va);
    read_rows(vs1, vb);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // slots read: refill them
    if (st + 1 < n_pairs) {
      const int pn = p + 1 == n_pairs ? 0 : p + 1;
      load_chunk(kbase, kss2, kofs, 2 * pn, lk0);
      load_chunk(kbase, kss2, kofs, 2 * pn + 1, lk1);
      load_chunk(vbase, vss2, vofs, 2 * pn, lv0);
      load_chunk(vbase, vss2, vofs, 2 * pn + 1, lv1);
    }
    const int kb0 = 32 * p + 4 * q;
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const f32x4 pa = product(va, dop[u]);
      const f32x4 pb = product(vb, dop[u]);
      const uint64_t wa = win_words(u, sa[u], pa, kb0), wb = win_words(u, sb[u], pb, kb0 + 16);
      const u32x4 sq = {(uint32_t)wa, (uint32_t)(wa >> 32), (uint32_t)wb, (uint32_t)(wb >> 32)};
      const V8 sop = __builtin_bit_cast(V8, sq);
#pragma unroll
      for (int s = 0; s < C::NV; ++s) {
        const s16x4 kk[2] = {ta[s], tb[s]};
        dqacc[u][s] = M::mfma16(__builtin_bit_cast(V8, kk), sop, dqacc[u][s]);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);

#pragma unroll
  for (int u = 0; u < G; ++u) {
    // the 16-row group's non-finite flag (see band_dq_kernel)
    const int g16 = 2 * gq + u;
    const bool bad = wave_any(!sum_finite(dqacc[u]));
    if (lane == 0 && g16 < A.ng) A.flags[(int64_t)bh * A.ng + g16] = bad ? 1 : 0;
    const int i = r0 + 16 * u + n;
    if (i < A.q_len) {
      uint16_t* dqr = A.dq + (int64_t)b * A.dqsb + (int64_t)h * A.dqsh + (int64_t)i * A.dqss;
#pragma unroll
      for (int t = 0; t < C::NV / 2; ++t) {
        V8 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ov[e] = (typename M::s)(dqacc[u][2 * t][e] * A.sm_scale);
          ov[4 + e] = (typename M::s)(dqacc[u][2 * t + 1][e] * A.sm_scale);
        }
        *(V8*)(dqr + C::CW * q + 8 * t) = ov;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Band-gathered dK / dV: one wave per (batch, kv head, 16-key block
// [u0, u0 + 16)).  Entry j's key is nondecreasing in the row (the window
// start, the spacing and both interpolated terms of the recipe never
// decrease), so for each query head of the kv group and each entry j the
// rows whose key of entry j lies in the block form one range, which one lane
// finds by binary search (lane r takes entry (r + rot) mod 64, see below).
// The ranges are packed back to back in lane order and walked 32 rows at a
// time (a step may hold rows of several entries): each slot row's Q and dO
// row is staged in LDS by buffer_load ... lds with per-lane row offsets
// (empty slot rows read as zeros), its delta and lse2 by a one-dword DMA,
// then
//   S = Q K^T, dP = dO V^T   2 x D/32 MFMAs each (A = Q / dO rows from LDS,
//                            B = the block's K / V in registers)
//   P = exp2(S scale log2e - lse2), dS = P (dP - delta) on the (row, key)
//   pairs where the key is the row's entry j and not past the row (one key
//   per row)
//   dV^T += dO^T P, dK^T += Q^T dS   D/16 MFMAs each over the 32 rows (A =
//                            dO^T / Q^T read transposed from the same slots)
// dK = scale dK^T^T.  Each (row, entry) pair lands in exactly one block and
// one step, as in the reference's dK/dV loop (:168-233 accumulates the same
// pairs); every gradient row is accumulated in a fixed order (by one wave,
// or by the parts of a split block added in part order): deterministic, no
// atomics on gradients.
//
// Schedule.  A row's Q and dO serve every block holding one of its keys, so
// the blocks one XCD runs at a time should be neighbours (one L2): blocks go
// to the eight XCDs in chunks of A.kchunk consecutive blocks, round robin
// (with whole kv heads per XCD, batch * kv heads a multiple of 8, one chunk
// per XCD, each a contiguous range; otherwise chunks of 8 blocks, which
// balance the heavy low blocks over the XCDs), and each block starts its
// walk at entry rot, a little more than 64 / (resident waves per XCD) of an
// entry further per block dispatched on the XCD, so the resident blocks walk
// neighbouring entries (the rotation of band_rows; none for a grid of a few
// rounds, band_rotation).  At the last layer of a pattern key block 0 takes
// far more rows than the rest (entry 0 of the heads with small interpolation weight
// stays in it for thousands of rows), so the host splits blocks
// 0 .. split_blocks - 1 (block 0) over split_parts waves each: each part
// walks a fixed range of the block's steps (unrotated), stores float32 sums,
// and the part that arrives last (an atomic counter) adds the parts in part
// order and writes the block, so results do not depend on which wave is
// last.
//
// WIN: interpolation weight 0 (layer 0, a sliding window).  Key u is
// attended by rows u .. u + w - 1, so the block's rows are the one range
// [u0, u0 + 15 + w) (clipped to q_len), walked once per query head, and a
// slot row keeps every block key of its window (key <= row < key + w)
// instead of the one key of an entry.

template <int D, Elem E, bool WIN = false>
__global__ __launch_bounds__(64, 2) void band_dkdv_kernel(BwdArgs A, const float* lse2) {
  using M = MmaT<E>;
  using V8 = typename M::v8;
  using C = BandCfg<D>;
  constexpr int ROWS = 32;                // query rows per step
  constexpr int SLOT2 = ROWS * D;         // elements per Q or dO slot
  constexpr int SL = ROWS * C::CPR / 64;  // DMA instructions per slot
  __shared__ __attribute__((aligned(1024))) uint16_t qsl[SLOT2];
  __shared__ __attribute__((aligned(1024))) uint16_t osl[SLOT2];
  __shared__ __attribute__((aligned(256))) float lsl[64];  // delta, lse2 of the slot rows
  lds_u16* const lq = (lds_u16*)qsl;
  lds_u16* const lo = (lds_u16*)osl;

  // ---- work item: the first n_extra workgroups take parts 1 .. split_parts
  // - 1 of the split blocks; then slot k of XCD x takes block
  // (k / chunk * 8 + x) * chunk + k % chunk (part 0 if split)
  const int bid = blockIdx.x;
  int g, part = 0;
  if (bid < A.n_extra) {
    const int n_split = A.n_bkv * A.split_blocks;
    if (bid >= n_split * (A.split_parts - 1)) return;
    part = 1 + bid / n_split;
    const int sb = bid % n_split;  // (split block, b kv head), blocks outermost
    g = (sb % A.n_bkv) * A.nkb16 + sb / A.n_bkv;
  } else {
    const int bj = bid - A.n_extra;  // n_extra is a multiple of 8: same XCD
    const int kx = bj >> 3;
    g = ((kx / A.kchunk) * 8 + (bj & 7)) * A.kchunk + kx % A.kchunk;
    if (g >= A.n_kblk) return;
  }
  const int bkv = g / A.nkb16, kb = g % A.nkb16;
  const bool split = A.split_parts > 1 && kb < A.split_blocks;
  // entry rotation (as in band_rows): lane r of the walk holds entry
  // (r + rot) mod 64, rot growing by A.rot_dkdv 64ths of an entry per block
  // dispatched on the XCD (launch_band_dkdv picks the rate), so the blocks
  // resident at once walk neighbouring entries and share Q / dO rows in L2.
  // The parts of a split block walk one sequence: no rotation there.
  const int rot =
      split || WIN ? 0
                   : (int)(((unsigned)((bid - A.n_extra) >> 3) * (unsigned)A.rot_dkdv / 64u) & 63u);
  const int kvh = bkv % A.Hkv, b = bkv / A.Hkv;
  const int u0 = 16 * kb;

  const int lane = threadIdx.x;
  const int n = lane & 15, q = lane >> 4;
  const int key = u0 + n;
  const bool key_ok = key < A.kv_len;

  // the block's K and V as B operands: key n, dims 32 s + 8 q .. + 8
  V8 kop[C::NS], vop[C::NS];
  {
    const uint16_t* kr = A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh + (int64_t)key * A.kss;
    const uint16_t* vr = A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh + (int64_t)key * A.vss;
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
      u32x4 kraw = {0u, 0u, 0u, 0u}, vraw = {0u, 0u, 0u, 0u};
      if (key_ok) {
        kraw = *(const u32x4*)(kr + 32 * s + 8 * q);
        vraw = *(const u32x4*)(vr + 32 * s + 8 * q);
      }
      kop[s] = __builtin_bit_cast(V8, kraw);
      vop[s] = __builtin_bit_cast(V8, vraw);
    }
  }

  const int qss2 = (int)A.qss * 2, oss2 = (int)A.doss * 2;
  // DMA t, lane l fills slot row R_t = (64 t + l) / CPR at physical chunk
  // l % CPR, from logical chunk kswz(R_t, l % CPR) of the row the step puts
  // there (fetched from the lane holding slot row R_t)
  int dmar[SL], cofs[SL];
#pragma unroll
  for (int t = 0; t < SL; ++t) {
    const int R = (64 * t + lane) / C::CPR;
    dmar[t] = 4 * R;
    cofs[t] = 16 * kswz<D>(R, lane % C::CPR);
  }
  // row reads (A operand of S and dP) of chunk c (slot rows 16 c .. + 15):
  // lane (m = n, q) reads slot row 16 c + n, dims 32 s + 8 q .. + 8
  int rrd[C::NS];
#pragma unroll
  for (int s = 0; s < C::NS; ++s) rrd[s] = n * C::ROWB + 16 * kswz<D>(n, 4 * s + q);
  // transposed reads (A operand of dV^T, dK^T) for slice s of chunk c: lane
  // x of its 16-lane group reads slot row 16 c + 4 q + x/4, dims
  // CW (x%4) + 4 s .. + 3 (the swizzle of row 16 c + r is that of row r)
  int trd[C::NV];
#pragma unroll
  for (int s = 0; s < C::NV; ++s) {
    const int R = 4 * q + (n >> 2), dim0 = C::CW * (n & 3) + 4 * s;
    trd[s] = R * C::ROWB + 16 * kswz<D>(R, dim0 >> 3) + 2 * (dim0 & 7);
  }
  constexpr int CHB = 16 * C::ROWB;  // bytes of one 16-row chunk

  f32x4 dkacc[C::NV], dvacc[C::NV];
#pragma unroll
  for (int s = 0; s < C::NV; ++s) dkacc[s] = dvacc[s] = f32x4{};
  const float scale2 = A.scale_log2;
  constexpr int kWaitLds = 0xC07F;  // lgkmcnt(0)
  // Each step issues, in order, its successor's Q DMAs (SL), dO DMAs (SL)
  // and delta / lse2 DMA (1), each after the step's reads of that buffer.
  // Loads complete in order, so: Q of this step is in LDS once at most
  // SL + 1 loads (its dO and delta / lse2) are outstanding; dO once at most
  // SL + 1 (its delta / lse2, the next Q); delta / lse2 once at most 2 SL.
  constexpr int kWaitRows = (0xF70 & ~0xF) | ((SL + 1) & 0xF) | (((SL + 1) >> 4) << 14);
  constexpr int kWaitStats = (0xF70 & ~0xF) | ((2 * SL) & 0xF) | (((2 * SL) >> 4) << 14);
  // a buffer offset past every resource used here (num_records < 2^31 - 16),
  // so a DMA lane without a row reads zeros and fetches nothing
  constexpr int kOob = 0x7ffffff0;
  const int slot_row = lane & 31;
  const int lse_off = (int)((const char*)lse2 - (const char*)A.delta);

  // lane r of head h, entry j = (r + rot) mod 64: rows [r0, r0 + len) whose
  // key of entry j lies in the block (rows before u0 cannot use a key >= u0);
  // the ranges are packed back to back in lane order: lane r's rows are
  // positions [cum, cum + len) of one sequence, walked 32 positions per step;
  // returns the sequence length
  auto head_ranges = [&](int h, int& r0, int& len, int& cum) {
    const HeadWeights hw = head_weights(A.pc, h);
    auto key_at = [&](int i, int j) {
      const RowParams rp = row_params(A.pc, i);
      return interp_index(oversized(rp, j), oversized(rp, j + 1), hw);
    };
    r0 = 0;
    len = 0;
    const int ej = (lane + rot) & 63;
    if constexpr (WIN) {
      r0 = u0;
      len = lane == 0 ? max(min(u0 + 15 + A.pc.w, A.q_len) - u0, 0) : 0;
    } else if (ej < A.pc.w) {
      int a0 = u0, a1 = A.q_len;  // first row >= u0 with key >= u0
      while (a0 < a1) {
        const int mid = (a0 + a1) >> 1;
        if (key_at(mid, ej) >= u0) a1 = mid; else a0 = mid + 1;
      }
      int c0 = a0, c1 = A.q_len;  // first row with key >= u0 + 16
      while (c0 < c1) {
        const int mid = (c0 + c1) >> 1;
        if (key_at(mid, ej) >= u0 + 16) c1 = mid; else c0 = mid + 1;
      }
      r0 = a0;
      len = c0 - a0;
    }
    cum = len;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(cum, off, 64);
      if (lane >= off) cum += t;
    }
    const int total = __builtin_amdgcn_readlane(cum, 63);
    cum -= len;
    return total;
  };
  // a split block's part takes steps [s_lo, s_hi) of the group's heads' step
  // sequences laid end to end
  int s_lo = 0, s_hi = 0x7fffffff;
  if (split) {
    int64_t steps = 0;
    for (int hg = 0; hg < A.groups; ++hg) {
      int r0, len, cum;
      steps += (head_ranges(kvh * A.groups + hg, r0, len, cum) + ROWS - 1) / ROWS;
    }
    s_lo = (int)(steps * part / A.split_parts);
    s_hi = (int)(steps * (part + 1) / A.split_parts);
  }

  int s_base = 0;  // steps of the earlier heads
  for (int hg = 0; hg < A.groups; ++hg) {
    const int h = kvh * A.groups + hg;
    const HeadWeights hw = head_weights(A.pc, h);
    auto key_at = [&](int i, int j) {
      const RowParams rp = row_params(A.pc, i);
      return interp_index(oversized(rp, j), oversized(rp, j + 1), hw);
    };
    int r0, len, cum;
    const int total = head_ranges(h, r0, len, cum);
    const int steps_h = (total + ROWS - 1) / ROWS;
    const int ls0 = min(max(s_lo - s_base, 0), steps_h), ls1 = min(max(s_hi - s_base, 0), steps_h);
    s_base += steps_h;
    if (ls0 >= ls1) continue;
    const int p_first = ROWS * ls0, p_end = min(total, ROWS * ls1);
    const uint64_t live = __builtin_amdgcn_ballot_w64(len > 0);
    // row and walk lane of slot row (lane % 32) in the step at position P
    // (row -1: none; the lane's entry is (lane + rot) mod 64); e is the first
    // live lane reaching past P on entry, the first reaching past P + 32 on
    // return
    auto map_step = [&](int P, int& e, int& row, int& ent) {
      row = -1;
      ent = 0;
      while (e < 64) {
        const int ce = __builtin_amdgcn_readlane(cum, e);
        if (ce >= P + ROWS) break;
        const int le = __builtin_amdgcn_readlane(len, e);
        const int re = __builtin_amdgcn_readlane(r0, e);
        const int d = P + slot_row - ce;
        if ((uint32_t)d < (uint32_t)le) {
          row = re + d;
          ent = e;
        }
        if (ce + le > P + ROWS) break;
        const uint64_t rest = e >= 63 ? 0ull : (live & (~0ull << (e + 1)));
        e = rest ? (int)__builtin_ctzll(rest) : 64;
      }
    };

    const char* const qbase = (const char*)(A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh);
    const char* const obase = (const char*)(A.dout + (int64_t)b * A.dosb + (int64_t)h * A.dosh);
    const char* const sbase = (const char*)(A.delta + ((int64_t)b * A.H + h) * A.qpad);
    const __amdgpu_buffer_rsrc_t qrs =
        __builtin_amdgcn_make_buffer_rsrc((void*)qbase, (short)0, A.q_len * qss2, 0x00020000);
    const __amdgpu_buffer_rsrc_t ors =
        __builtin_amdgcn_make_buffer_rsrc((void*)obase, (short)0, A.q_len * oss2, 0x00020000);
    // delta row of (b, h) and, lse_off bytes further, its lse2 row
    const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)sbase, (short)0, lse_off + 4 * A.qpad, 0x00020000);
    // Q or dO rows of the step whose slot rows hold `row` -> slot dst (after
    // the step's reads of dst)
    auto issue_rows = [&](__amdgpu_buffer_rsrc_t rs, int ss2, int row, lds_u16* dst) {
      // (a fixed size: hipcc drops the kernel's host stub when a lambda here
      // declares an array whose size depends on D)
      static_assert(SL <= 8, "at most 8 DMAs per slot");
      int ofs[8];
#pragma unroll
      for (int t = 0; t < SL; ++t) {
        const int rr = __builtin_amdgcn_ds_bpermute(dmar[t], row);
        ofs[t] = rr >= 0 ? rr * ss2 + cofs[t] : kOob;
      }
      __builtin_amdgcn_s_waitcnt(kWaitLds);  // the slot's reads are done
#pragma unroll
      for (int t = 0; t < SL; ++t)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + 512 * t), 16, ofs[t], 0,
                                                 0, 0);
    };
    // delta (lanes 0..31) and lse2 (lanes 32..63) of the step's rows -> lsl
    auto issue_stats = [&](int row) {
      const int ofs = row >= 0 ? 4 * row + (lane >= 32 ? lse_off : 0) : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(srs, (lds_void*)lsl, 4, ofs, 0, 0, 0);
    };

    // the first live entry reaching past the part's first position
    int e = (int)__builtin_ctzll(__builtin_amdgcn_ballot_w64(len > 0 && cum + len > p_first));
    int row_c, ent_c;
    map_step(p_first, e, row_c, ent_c);
    issue_rows(qrs, qss2, row_c, lq);
    issue_rows(ors, oss2, row_c, lo);
    __builtin_amdgcn_s_waitcnt(kWaitLds);  // the last head's stats reads are done
    issue_stats(row_c);
    for (int P = p_first; P < p_end; P += ROWS) {
      int row_n = -1, ent_n = 0;
      if (P + ROWS < p_end) map_step(P + ROWS, e, row_n, ent_n);
      // the key of slot row (lane % 32), -1 when masked or empty
      int rkey = -1;
      if constexpr (WIN) {
        rkey = row_c;
      } else if (row_c >= 0) {
        const int kk = key_at(row_c, (ent_c + rot) & 63);
        rkey = kk <= row_c ? kk : -1;
      }

      __builtin_amdgcn_s_waitcnt(kWaitRows);  // this step's Q is in LDS
      f32x4 sacc[2];
      s16x4 qt[2][C::NV];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        V8 qa[C::NS];
#pragma unroll
        for (int s = 0; s < C::NS; ++s)
          qa[s] = *(const V8*)((const char*)qsl + c * CHB + rrd[s]);
        sacc[c] = M::mfma16(qa[0], kop[0], f32x4{});
#pragma unroll
        for (int s = 1; s < C::NS; ++s) sacc[c] = M::mfma16(qa[s], kop[s], sacc[c]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int s = 0; s < C::NV; ++s)
          qt[c][s] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4*)((const char*)qsl + c * CHB + trd[s]));
      issue_rows(qrs, qss2, row_n, lq);

      __builtin_amdgcn_s_waitcnt(kWaitRows);  // this step's dO is in LDS
      f32x4 pacc[2];
      s16x4 ot[2][C::NV];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        V8 oa[C::NS];
#pragma unroll
        for (int s = 0; s < C::NS; ++s)
          oa[s] = *(const V8*)((const char*)osl + c * CHB + rrd[s]);
        pacc[c] = M::mfma16(oa[0], vop[0], f32x4{});
#pragma unroll
        for (int s = 1; s < C::NS; ++s) pacc[c] = M::mfma16(oa[s], vop[s], pacc[c]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int s = 0; s < C::NV; ++s)
          ot[c][s] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4*)((const char*)osl + c * CHB + trd[s]));
      issue_rows(ors, oss2, row_n, lo);

      __builtin_amdgcn_s_waitcnt(kWaitStats);  // this step's delta / lse2 are in LDS
      f32x4 l2v[2], dlv[2];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        dlv[c] = *(const f32x4*)(lsl + 16 * c + 4 * q);
        l2v[c] = *(const f32x4*)(lsl + 32 + 16 * c + 4 * q);
      }
      __builtin_amdgcn_s_waitcnt(kWaitLds);  // stats read: refill them
      issue_stats(row_n);

      // P and dS where the row's key is this lane's key: lane (key n, q)
      // holds slot rows 16 c + 4 q + e, which are k-slots 8 q + 4 c + e of
      // the products over rows
      uint32_t pw[4], sw[4];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float pv[4], dv[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const int rk = __builtin_amdgcn_ds_bpermute(4 * (16 * c + 4 * q + e2), rkey);
          // (WIN: rk is the slot row, -1 for none)
          const bool has = WIN ? rk >= 0 && key <= rk && key > rk - A.pc.w : rk == key;
          const float p =
              __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[c][e2], scale2, -l2v[c][e2]));
          pv[e2] = has ? p : 0.f;
          dv[e2] = has ? p * (pacc[c][e2] - dlv[c][e2]) : 0.f;
        }
        pw[2 * c] = M::pack2(pv[0], pv[1]);
        pw[2 * c + 1] = M::pack2(pv[2], pv[3]);
        sw[2 * c] = M::pack2(dv[0], dv[1]);
        sw[2 * c + 1] = M::pack2(dv[2], dv[3]);
      }
      const u32x4 pq = {pw[0], pw[1], pw[2], pw[3]};
      const u32x4 sq = {sw[0], sw[1], sw[2], sw[3]};
#pragma unroll
      for (int s = 0; s < C::NV; ++s) {
        const s16x4 oo[2] = {ot[0][s], ot[1][s]};
        dvacc[s] =
            M::mfma16(__builtin_bit_cast(V8, oo), __builtin_bit_cast(V8, pq), dvacc[s]);
        const s16x4 qq[2] = {qt[0][s], qt[1][s]};
        dkacc[s] =
            M::mfma16(__builtin_bit_cast(V8, qq), __builtin_bit_cast(V8, sq), dkacc[s]);
      }
      row_c = row_n;
      ent_c = ent_n;
    }
    // the last step's (empty) refills have landed before the next head's
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  }

  // ---- a split block: every part stores its float32 sums; the part that
  // arrives last adds the parts in part order (a fixed order whichever wave
  // is last) and writes the block
  if (split) {
    constexpr int PART = 2 * C::NV * 4 * 64;  // floats per part
    const int sb = bkv * A.split_blocks + kb;
    float* const pb = A.part_buf + (int64_t)sb * A.split_parts * PART;
    float* const mine = pb + (int64_t)part * PART;
#pragma unroll
    for (int s = 0; s < C::NV; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        mine[((0 * C::NV + s) * 4 + e) * 64 + lane] = dkacc[s][e];
        mine[((1 * C::NV + s) * 4 + e) * 64 + lane] = dvacc[s][e];
      }
    __threadfence();  // the sums are visible to the other XCDs before arriving
    int arrived = 0;
    if (lane == 0) arrived = atomicAdd(&A.part_cnt[sb], 1);
    arrived = __shfl(arrived, 0, 64);
    if (arrived != A.split_parts - 1) return;
    __threadfence();  // the other parts' sums, not stale copies
#pragma unroll
    for (int s = 0; s < C::NV; ++s) dkacc[s] = dvacc[s] = f32x4{};
    for (int pp = 0; pp < A.split_parts; ++pp) {
      const float* src = pb + (int64_t)pp * PART;
#pragma unroll
      for (int s = 0; s < C::NV; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dkacc[s][e] += src[((0 * C::NV + s) * 4 + e) * 64 + lane];
          dvacc[s][e] += src[((1 * C::NV + s) * 4 + e) * 64 + lane];
        }
    }
  }

  // ---- the block's non-finite flag (bwd_fix_kernel recomputes it)
  {
    const bool bad = wave_any(!sum_finite(dkacc) || !sum_finite(dvacc));
    if (lane == 0) A.flags[A.n_qflags + g] = bad ? 1 : 0;
  }
  // ---- dK = scale dK^T^T, dV = dV^T^T: lane (key n, q) holds dims
  // CW q + 4 s + e of key u0 + n
  if (key_ok) {
    uint16_t* dkr = A.dk + (int64_t)b * A.dksb + (int64_t)kvh * A.dksh + (int64_t)key * A.dkss;
    uint16_t* dvr = A.dv + (int64_t)b * A.dvsb + (int64_t)kvh * A.dvsh + (int64_t)key * A.dvss;
#pragma unroll
    for (int t = 0; t < C::NV / 2; ++t) {
      V8 kv, vv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kv[e] = (typename M::s)(dkacc[2 * t][e] * A.sm_scale);
        kv[4 + e] = (typename M::s)(dkacc[2 * t + 1][e] * A.sm_scale);
        vv[e] = (typename M::s)dvacc[2 * t][e];
        vv[4 + e] = (typename M::s)dvacc[2 * t + 1][e];
      }
      *(V8*)(dkr + C::CW * q + 8 * t) = kv;
      *(V8*)(dvr + C::CW * q + 8 * t) = vv;
    }
  }
}

template <Elem E>
static void launch_band_dkdv_elem(const BwdArgs& a, int head_dim, dim3 grid, const float* lse2,
                                  hipStream_t stream) {
  // a sliding window at interpolation weight 0
  const bool win = a.pc.a == 0.0f;
  if (head_dim == 128) {
    if (win)
      band_dkdv_kernel<128, E, true><<<grid, 64, 0, stream>>>(a, lse2);
    else
      band_dkdv_kernel<128, E><<<grid, 64, 0, stream>>>(a, lse2);
  } else {
    if (win)
      band_dkdv_kernel<64, E, true><<<grid, 64, 0, stream>>>(a, lse2);
    else
      band_dkdv_kernel<64, E><<<grid, 64, 0, stream>>>(a, lse2);
  }
}

hipError_t launch_band_dkdv(const BwdArgs& a, int head_dim, const float* lse2,
                            hipStream_t stream) {
  if (a.n_kblk <= 0 || a.kchunk <= 0) return hipSuccess;
  const int64_t chunks = (a.n_kblk + 8 * (int64_t)a.kchunk - 1) / (8 * (int64_t)a.kchunk);
  const dim3 grid((unsigned)(a.n_extra + chunks * 8 * a.kchunk));
  // Entry rotation: 19/64 (D = 128: 256 resident waves per XCD) or 12/64
  // (D = 64: 384), a little ahead of the dispatch rate; none for a grid of
  // a few rounds whose heads' Q and dO rows exceed L2 (band_rotation).  Same
  // box, without against with: B=1 H=4 L=32768 D=128 (four rounds) backward
  // -4% at layer 4, -9% at layer 7, B=1 H=2 L=65536 -5.5%; at eight rounds
  // (H=8) +1.4%, at 32 (H=32) +4.3%.  A few-round rate of 3/64 (the
  // forward's) was 3-10% slower than none here.
  BwdArgs r = a;
  r.rot_dkdv = band_rotation(a.n_kblk, head_dim == 128 ? 256 : 384,
                             (int64_t)a.q_len * 4 * head_dim, head_dim == 128 ? 19 : 12, 0);
  if (a.elem == (int)Elem::f16)
    launch_band_dkdv_elem<Elem::f16>(r, head_dim, grid, lse2, stream);
  else
    launch_band_dkdv_elem<Elem::bf16>(r, head_dim, grid, lse2, stream);
  return hipGetLastError();
}

template <int D, bool PREP, Elem E>
static void launch_band_dq_d(const BwdArgs& a, dim3 grid, const float* lse2, hipStream_t stream) {
  // a sliding window at interpolation weight 0; K and V DMA skipping from
  // interpolation weight 1/2 on, as for the forward
  if (a.pc.a == 0.0f) {
    // 32-row groups (window_dq_kernel), XCD-contiguous like the 16-row grid
    const int64_t n2 = (int64_t)a.B * a.H * ((a.q_len + 31) / 32);
    window_dq_kernel<D, PREP, E><<<dim3((unsigned)(8 * ((n2 + 7) / 8))), 64, 0, stream>>>(a, lse2);
  } else if (a.pc.a >= 0.5f)
    band_dq_kernel<D, true, PREP, E><<<grid, 64, 0, stream>>>(a, lse2);
  else
    band_dq_kernel<D, false, PREP, E><<<grid, 64, 0, stream>>>(a, lse2);
}

template <Elem E>
static void launch_band_dq_elem(const BwdArgs& a, int head_dim, dim3 grid, const float* lse2,
                                bool prep, hipStream_t stream) {
  if (head_dim == 128) {
    if (prep)
      launch_band_dq_d<128, true, E>(a, grid, lse2, stream);
    else
      launch_band_dq_d<128, false, E>(a, grid, lse2, stream);
  } else {
    if (prep)
      launch_band_dq_d<64, true, E>(a, grid, lse2, stream);
    else
      launch_band_dq_d<64, false, E>(a, grid, lse2, stream);
  }
}

hipError_t launch_band_dq(const BwdArgs& a, int head_dim, const float* lse2, bool prep,
                          hipStream_t stream) {
  if (a.n_groups <= 0) return hipSuccess;
  dim3 grid((unsigned)(8 * a.per_xcd));
  // Entry rotation: 19/64 (D = 128: 256 resident waves per XCD) or 12/64
  // (D = 64: 512), a little ahead of the dispatch rate 64 / 256 = 16/64 or
  // 8/64 (19/64 measured 1-4% faster than 16/64 at B=1 H=8 L=131072 layers
  // 4 and 7, unchanged at B=1 H=32 L=32768; 9/64 at D = 64 within 1% of
  // 12/64); none for a grid of a few rounds whose heads' K and V exceed L2
  // (band_rotation, measured with the dK / dV's in launch_band_dkdv)
  BwdArgs r = a;
  r.rot_dq = band_rotation(a.n_groups, head_dim == 128 ? 256 : 512,
                           (int64_t)a.kv_len * 4 * head_dim, head_dim == 128 ? 19 : 12, 0);
  if (a.elem == (int)Elem::f16)
    launch_band_dq_elem<Elem::f16>(r, head_dim, grid, lse2, prep, stream);
  else
    launch_band_dq_elem<Elem::bf16>(r, head_dim, grid, lse2, prep, stream);
  return hipGetLastError();
}

}  // namespace esa
