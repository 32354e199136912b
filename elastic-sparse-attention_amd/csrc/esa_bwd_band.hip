// Band-gathered dQ of the elastic prefill backward (gfx950).
//
// Replaces the dQ half of the reference's Triton backward
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
// key) pair contributes once, as in :191-228; dK and dV come from
// dkdv_kernel (esa_bwd.hip).  Operand layouts: esa_band.hpp.
#include "esa_band.hpp"

namespace esa {

template <int D>
__global__ __launch_bounds__(64, 2) void band_dq_kernel(BwdArgs A, const float* lse2) {
  using C = BandCfg<D>;
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
  bf16x8 qop[C::NS], dop[C::NS];
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
      qop[s] = __builtin_bit_cast(bf16x8, qraw);
      dop[s] = __builtin_bit_cast(bf16x8, draw);
    }
  }
  float l2 = 0.f, dl = 0.f;
  if (row_ok) {
    const int64_t at = ((int64_t)b * A.H + h) * A.q_len + i;
    l2 = lse2[at];
    dl = A.delta[at];
  }

  int kreg[16], info[16];
  band_rows(A.pc, h, i, row_ok, q, kreg, info);

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
  // band's W rows (rows past the band read as zeros without a fetch)
  auto load_rows = [&](const char* base, int ss2, const int* ofs, int bi, lds_u16* dst) {
    const int lo = bi & 0xffffff, wdt = (int)((uint32_t)bi >> 24);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(base + (int64_t)lo * ss2), (short)0, min(wdt, 16) * ss2, 0x00020000);
#pragma unroll
    for (int t = 0; t < C::VLOADS; ++t)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + 512 * t), 16, ofs[t], 0, 0,
                                               0);
  };
  auto load_k = [&](int bi, lds_u16* dst) { load_rows(kbase, kss2, kofs, bi, dst); };
  auto load_v = [&](int bi, lds_u16* dst) { load_rows(vbase, vss2, vofs, bi, dst); };

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
  auto read_rows = [&](const uint16_t* src, bf16x8 (&op)[C::NS]) {
#pragma unroll
    for (int s = 0; s < C::NS; ++s) op[s] = *(const bf16x8*)((const char*)src + rrd[s]);
  };
  auto read_tr = [&](const uint16_t* src, s16x4 (&op)[C::NV]) {
#pragma unroll
    for (int s = 0; s < C::NV; ++s)
      op[s] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((const char*)src + trd[s]));
  };
  auto product = [&](const bf16x8 (&a)[C::NS], const bf16x8 (&bop)[C::NS]) {
    f32x4 acc = mfma16(a[0], bop[0], f32x4{});
#pragma unroll
    for (int s = 1; s < C::NS; ++s) acc = mfma16(a[s], bop[s], acc);
    return acc;
  };

  const float scale2 = A.scale_log2;
  // dS of this row's key in chunk [c0, c0 + 16) of a band, as bf16 at the
  // key's register slot of the lane holding it (0 elsewhere)
  auto ds_word = [&](const f32x4& sacc, const f32x4& pacc, int key, int c0) -> uint64_t {
    const int d = key - c0;
    const bool has = key >= 0 && (uint32_t)d < 16u && (d >> 2) == q;
    const int e = d & 3;
    const float s01 = (e & 1) ? sacc[1] : sacc[0];
    const float s23 = (e & 1) ? sacc[3] : sacc[2];
    const float dp01 = (e & 1) ? pacc[1] : pacc[0];
    const float dp23 = (e & 1) ? pacc[3] : pacc[2];
    const float s = (e & 2) ? s23 : s01;
    const float dp = (e & 2) ? dp23 : dp01;
    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s, scale2, -l2));
    const uint32_t w = (uint32_t)f32_to_bf16_bits(p * (dp - dl));
    return has ? ((uint64_t)w << (16 * e)) : 0ull;
  };

  f32x4 dqacc[C::NV];
#pragma unroll
  for (int s = 0; s < C::NV; ++s) dqacc[s] = f32x4{};
  // dQ^T += K^T dS^T over two bands' keys
  auto dq_step = [&](const s16x4 (&ta)[C::NV], const s16x4 (&tb)[C::NV], uint64_t wa,
                     uint64_t wb) {
    const u32x4 sq = {(uint32_t)wa, (uint32_t)(wa >> 32), (uint32_t)wb, (uint32_t)(wb >> 32)};
    const bf16x8 sop = __builtin_bit_cast(bf16x8, sq);
#pragma unroll
    for (int s = 0; s < C::NV; ++s) {
      const s16x4 kk[2] = {ta[s], tb[s]};
      dqacc[s] = mfma16(__builtin_bit_cast(bf16x8, kk), sop, dqacc[s]);
    }
  };

  // ---- band pairs: per pair, K reads, then K of the next pair; V reads,
  // then V of the next pair (so before each wait exactly 2 VLOADS newer
  // loads may be in flight)
  constexpr int kWaitPair = (0xF70 & ~0xF) | ((2 * C::VLOADS) & 0xF) |
                            (((2 * C::VLOADS) >> 4) << 14);  // vmcnt(2 VLOADS)
  constexpr int kWaitLds = 0xC07F;                           // lgkmcnt(0)
  const int lane_key = 4 * n;
  {
    const int i0 = __builtin_amdgcn_readlane(info[0], 0);
    const int i1 = __builtin_amdgcn_readlane(info[1], 0);
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
      const int ia = __builtin_amdgcn_readlane(info[ra], 16 * qj);
      const int ib = __builtin_amdgcn_readlane(info[rb], 16 * qj);
      int na, nb;
      if (rp < 7) {
        na = __builtin_amdgcn_readlane(info[ra + 2], 16 * qj);
        nb = __builtin_amdgcn_readlane(info[rb + 2], 16 * qj);
      } else {
        na = more ? __builtin_amdgcn_readlane(info[0], 16 * qj + 16) : 0;
        nb = more ? __builtin_amdgcn_readlane(info[1], 16 * qj + 16) : 0;
      }
      const bool live = (ia | ib) != 0;
      __builtin_amdgcn_s_waitcnt(kWaitPair);  // this pair's K is in LDS
      f32x4 sa, sb;
      s16x4 ta[C::NV], tb[C::NV];
      if (live) {
        {
          bf16x8 ka[C::NS], kb[C::NS];
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
      __builtin_amdgcn_s_waitcnt(kWaitPair);  // this pair's V is in LDS
      bf16x8 va[C::NS], vb[C::NS];
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
        const int addr = lane_key + 64 * qj;
        const int keya = __builtin_amdgcn_ds_bpermute(addr, kreg[ra]);
        const int keyb = __builtin_amdgcn_ds_bpermute(addr, kreg[rb]);
        const uint64_t wa = ds_word(sa, pa, keya, ia & 0xffffff);
        const uint64_t wb = ds_word(sb, pb, keyb, ib & 0xffffff);
        dq_step(ta, tb, wa, wb);
      }
    }
  }

  // ---- tail: keys of bands wider than 16, one 16-key chunk at a time (the
  // pair's second half is ks1 with dS = 0; ks1 holds finite rows)
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  int wmax = 0;
#pragma unroll
  for (int r = 0; r < 16; ++r) wmax = max(wmax, (int)((uint32_t)info[r] >> 24));
  for (int j = 0; j < 64 && wave_any(wmax > 16); ++j) {
    const int qj = j >> 4;
    int bi = 0, key = -1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if ((j & 15) == r) {
        bi = __builtin_amdgcn_readlane(info[r], 16 * qj);
        key = __builtin_amdgcn_ds_bpermute(lane_key + 64 * qj, kreg[r]);
      }
    }
    const int lo = bi & 0xffffff, wdt = (int)((uint32_t)bi >> 24);
    for (int c0 = lo + 16; c0 < lo + wdt; c0 += 16) {
      const int ci = c0 | (min(lo + wdt - c0, 16) << 24);
      __builtin_amdgcn_s_waitcnt(kWaitLds);
      load_k(ci, lk0);
      load_v(ci, lv0);
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      bf16x8 kt[C::NS], vt[C::NS];
      s16x4 tt[C::NV], tz[C::NV];
      read_rows(ks0, kt);
      read_rows(vs0, vt);
      read_tr(ks0, tt);
      read_tr(ks1, tz);
      const f32x4 st = product(kt, qop);
      const f32x4 pt = product(vt, dop);
      dq_step(tt, tz, ds_word(st, pt, key, c0), 0ull);
    }
  }

  // ---- dQ = scale * dQ^T^T: lane (n, q) holds dims CW q + 4 s + e of row n
  if (row_ok) {
    uint16_t* dqr = A.dq + (int64_t)b * A.dqsb + (int64_t)h * A.dqsh + (int64_t)i * A.dqss;
#pragma unroll
    for (int t = 0; t < C::NV / 2; ++t) {
      bf16x8 ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ov[e] = (__bf16)(dqacc[2 * t][e] * A.sm_scale);
        ov[4 + e] = (__bf16)(dqacc[2 * t + 1][e] * A.sm_scale);
      }
      *(bf16x8*)(dqr + C::CW * q + 8 * t) = ov;
    }
  }
}

hipError_t launch_band_dq(const BwdArgs& a, int head_dim, const float* lse2,
                          hipStream_t stream) {
  if (a.n_groups <= 0) return hipSuccess;
  dim3 grid((unsigned)(8 * a.per_xcd));
  if (head_dim == 128)
    band_dq_kernel<128><<<grid, 64, 0, stream>>>(a, lse2);
  else
    band_dq_kernel<64><<<grid, 64, 0, stream>>>(a, lse2);
  return hipGetLastError();
}

}  // namespace esa
