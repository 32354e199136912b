// Band-gathered forward over the elastic pattern (gfx950), prefill rows.
//
// Replaces the forward branch of the reference's per-token Triton kernel
// (elastic_sparse_attention.py:117-166) for query positions 0 .. q_len - 1,
// with the index list of every row regenerated on the device (the recipe of
// elastic_sparse_attention.py:482-535).
//
// Structure the kernel relies on: entry j of a row's index list (its "band")
// moves by 0 or 1 key from one row to the next (by 2 at a few rows of a head
// whose interpolation weight is 1/2), so across 16 consecutive rows band j
// spans at most 16 consecutive keys, rarely 17.  One wave owns
// 16 query rows (a group).  For each band it gathers the keys [lo_j, lo_j+16)
// (lo_j = the band's smallest valid key over the group; keys past the band's
// largest one read as zero and cost no traffic), computes the 16 x 16 scores
// with MFMA, keeps for each row only its own key of the band (exactly one
// per row and band, so no key is counted twice even where bands overlap),
// and accumulates P V with MFMA.  A band wider than 16 keys (not produced by
// the shapes measured, but allowed) gets its extra keys in a tail pass.
// Every group does the same number of bands, and waves share nothing: no
// barriers, no LDS shared between waves.
//
// Per band and wave:
//   S^T = K Q^T     D/32 x v_mfma_f32_16x16x32_{bf16,f16}; A = K rows read from
//                   LDS (lane m: key lo + m%16), B = Q held in registers for
//                   the whole group
//   select          each lane owns one row and 4 of the 16 keys; the lane
//                   holding the row's key of this band keeps its score, the
//                   row's 4 lanes share it with two lane swaps
//   softmax         online, log2 domain, one running-max update per band
//                   pair, lazy rescale (the running max moves only when a
//                   score exceeds it by more than 8)
//   O^T += V^T P^T  bands go in pairs (32 keys = one MFMA k-step): D/16 x
//                   v_mfma_f32_16x16x32_{bf16,f16}, A = V^T read with
//                   ds_read_b64_tr_b16 from row-major V rows in LDS, B = P
//                   straight from the select step
// K and V rows reach LDS by buffer_load ... lds, whole rows per 16 lanes:
// the L1 spends about a clock per (16-lane pass, cache line), so loading the
// MFMA operand straight into registers (16 key rows per pass) would cost 8x
// the L1 time.  Two K and two V slots per wave, refilled in one of two
// orders (VEARLY, picked by the host):
//   VEARLY    once a pair's K and V^T operands are in registers, the next
//             pair's K and V are requested together, so both have the whole
//             pair's scores, softmax and PV to land;
//   otherwise the next pair's K is requested once this pair's K operands are
//             in registers, its V once this pair's PV has read V.
//
// Operand layouts: esa_band.hpp.
#include "esa_band.hpp"
#include "esa_gather.hpp"

namespace esa {

// Band descriptor word: lo | W << 24 (W = keys from lo to the band's largest
// valid key, 0 for a band no row of the group uses); lo < 2^24 (host check).
//
// KSKIP: issue only the K DMAs that reach a band row (see load_rows).  Pays
// where many bands are narrower than 16 keys (the dilated, late layers);
// where nearly every band is 16 keys wide the run-time waits cost more than
// the DMAs saved, so the host picks it by the pattern's interpolation weight.
//
// POS: query rows at positions A.positions[r] (cache_position: a chunked
// prefill's rows p0 .. p0 + q_len - 1, or any positions).  A group whose rows
// sit at consecutive positions, all in [0, kv_len), runs as a prefill group
// from its first row's position (the bands only need consecutive positions,
// not a multiple of 16); any other group computes its rows one at a time
// with the per-row gather (gather_one_row_any: float32, the arithmetic of
// esa_elastic_fwd_rows).  Q, O and the log-sum-exp stay indexed by the row r.
// S: waves per group (S = 2 for grids that fit one round of resident
// workgroups, whose time is one group's whole walk): wave w walks the slots of
// lane groups 4 w / S .. 4 (w + 1) / S - 1 with slots of its own, and wave 0
// merges the other wave's softmax state (handed over through that wave's
// slots across one barrier) before the epilogue.
template <int D, bool KSKIP, bool VEARLY, Elem E, bool POS, int S = 1>
__global__ __launch_bounds__(64 * S, 2) void band_fwd_kernel(BandArgs A) {
  using C = BandCfg<D>;
  using M = MmaT<E>;
  using V8 = typename M::v8;
  static_assert(S == 1 || S == 2, "one or two waves per group");
  // K and V slots of the pair's two bands (separate objects, so the compiler
  // can tell reads of one slot from the direct loads into another), S sets
  __shared__ __attribute__((aligned(1024))) uint16_t ks0_[C::SLOT * S];
  __shared__ __attribute__((aligned(1024))) uint16_t ks1_[C::SLOT * S];
  __shared__ __attribute__((aligned(1024))) uint16_t vs0_[C::SLOT * S];
  __shared__ __attribute__((aligned(1024))) uint16_t vs1_[C::SLOT * S];
  const int wv = S > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;
  uint16_t* const ks0 = ks0_ + wv * C::SLOT;
  uint16_t* const ks1 = ks1_ + wv * C::SLOT;
  uint16_t* const vs0 = vs0_ + wv * C::SLOT;
  uint16_t* const vs1 = vs1_ + wv * C::SLOT;
  uint16_t* const slot[4] = {ks0, ks1, vs0, vs1};
  const int q0 = wv * (4 / S);  // this wave's first lane group of slots

  // ---- group: XCD x takes the contiguous range [x per, (x + 1) per)
  const int bid = blockIdx.x;
  const int g = (bid & 7) * A.per_xcd + (bid >> 3);
  if (g >= A.n_groups) return;
  const int bh = g / A.ng, gq = g % A.ng;
  const int h = bh % A.H, b = bh / A.H;
  const int kvh = h / A.groups;

  const int lane = S > 1 ? (int)(threadIdx.x & 63) : (int)threadIdx.x;
  const int n = lane & 15, q = lane >> 4;
  const int r = gq * 16 + n;  // this lane's query row (of q, o and lse)
  const bool row_ok = r < A.q_len;
  int i = r;  // its position
  if constexpr (POS) {
    int64_t p = row_ok ? A.positions[r] : 0;
    p = p < 0 ? p + A.kv_len : p;
    const bool in_range = p >= 0 && p < A.kv_len;
    // row 0 of a group always exists: the group's base position
    const int base = __builtin_amdgcn_readfirstlane((int)(in_range ? p : 0) - n);
    if (wave_any(row_ok && !(in_range && (int)p - n == base))) {
      // positions not consecutive (or out of range): the rows one at a time,
      // by the per-row gather, with the first K slot as its 384-float scratch
      // (the gather that holds few registers: this path must not raise the
      // kernel's register count)
      GatherArgs G{};
      G.q = A.q; G.k = A.k; G.v = A.v; G.o = A.o; G.lse = A.lse;
      G.qsb = A.qsb; G.qsh = A.qsh; G.qss = A.qss;
      G.ksb = A.ksb; G.ksh = A.ksh; G.kss = A.kss;
      G.vsb = A.vsb; G.vsh = A.vsh; G.vss = A.vss;
      G.osb = A.osb; G.osh = A.osh; G.oss = A.oss;
      G.lsb = A.lsb; G.lsh = A.lsh;
      // (the inputs' head dim: at a head dim padded up to the kernel's D the
      // rows hold d_real elements, and the gather reads and writes that many)
      G.H = A.H; G.groups = A.groups; G.q_len = A.q_len; G.kv_len = A.kv_len; G.D = A.d_real;
      G.sm_scale = A.sm_scale;
      G.elem = A.elem;
      G.src.w = A.pc.w; G.src.kv_len = A.kv_len; G.src.pc = A.pc;
      G.src.positions = A.positions;
      if (S > 1 && wv != 0) return;  // (every wave of the group takes this branch)
      for (int rr = 0; rr < 16 && gq * 16 + rr < A.q_len; ++rr)
        gather_one_row_any<E, true>(G, b, h, gq * 16 + rr, (float*)ks0, lane);
      return;
    }
    i = base + n;
  }

  // ---- slots to zeros once: rows a band does not fill keep finite values
  {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int c = 0; c < C::SLOT / 512; ++c) *(u32x4*)(slot[s] + (c * 64 + lane) * 8) = z;
  }

  // ---- Q as the B operand: row n, dims 32 s + 8 q .. + 8 for k-step s
  V8 qop[C::NS];
  {
    const uint16_t* qrow = A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)r * A.qss;
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row_ok && 32 * s + 8 * q < A.d_real) raw = *(const u32x4*)(qrow + 32 * s + 8 * q);
      qop[s] = __builtin_bit_cast(V8, raw);
    }
  }

  // ---- this row's keys of bands 16 q .. 16 q + 15 as offsets from the
  // bands' first keys (kd, byte r of word r / 4; 0xFF: no key), and the
  // group's band descriptors (slot (q, r)'s in lane 16 q + r of info1)
  uint32_t kd[4];
  int info1;
  // entry rotation, A.rot_rate 64ths of an entry per group dispatched on the
  // XCD (launch_band_fwd picks the rate)
  // (unsigned: the product wraps for grids near 2^31 blocks; only the value
  // mod 64 matters)
  band_rows(A.pc, h, i, row_ok, q, n,
            (int)(((unsigned)(bid >> 3) * (unsigned)A.rot_rate / 64u) & 63u), kd, info1);

  const char* const kbase = (const char*)(A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh);
  const char* const vbase = (const char*)(A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh);
  const int kss2 = (int)A.kss * 2, vss2 = (int)A.vss * 2;
  // LDS pointers of the slots, formed once (the DMA takes LDS addresses)
  lds_u16* const lk0 = (lds_u16*)ks0;
  lds_u16* const lk1 = (lds_u16*)ks1;
  lds_u16* const lv0 = (lds_u16*)vs0;
  lds_u16* const lv1 = (lds_u16*)vs1;

  // DMA t, lane l fills slot row R = (64 t + l) / CPR, physical chunk
  // l % CPR: its byte offset from the band's first row, fixed per lane
  // (a chunk past the inputs' head_dim gets an offset past every buffer's
  // num_records: it loads zeros)
  int kofs[C::VLOADS], vofs[C::VLOADS];
#pragma unroll
  for (int t = 0; t < C::VLOADS; ++t) {
    const int R = (64 * t + lane) / C::CPR, pc = lane % C::CPR;
    const int kc = kswz<D>(R, pc), vc = vswz<D>(R, pc);
    kofs[t] = 8 * kc < A.d_real ? R * kss2 + 16 * kc : 0x7ffffff0;
    vofs[t] = 8 * vc < A.d_real ? R * vss2 + 16 * vc : 0x7ffffff0;
  }
  // K or V rows of band info word `bi` -> slot dst, through a buffer resource
  // that starts at the band's first row and holds its W rows: rows past the
  // band fall outside num_records and read as zeros without a fetch.  V
  // takes only the ceil(W / RPI) DMAs that reach a band row (each DMA costs
  // the texture unit a full 64-lane transfer, rows past W included); its
  // slot rows past them keep an earlier band's rows, which meet p = 0 in PV
  // (0 * Inf = NaN for a non-finite one sends the group to the sanitised
  // rerun below, which gives the bits of a run without it).  K takes VLOADS
  // DMAs, or with KSKIP only those that reach a band row: K rows past the
  // band then keep older contents, whose scores belong to keys no row picks.
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
  auto load_k = [&](int bi, lds_u16* dst) { load_rows(kbase, kss2, kofs, bi, dst, !KSKIP); };
  auto load_v = [&](int bi, lds_u16* dst) { load_rows(vbase, vss2, vofs, bi, dst, false); };
  // s_waitcnt vmcnt(n) for a count known only at run time (0 .. 16)
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
      case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
      case 9: __builtin_amdgcn_s_waitcnt(0x0F79); break;
      case 10: __builtin_amdgcn_s_waitcnt(0x0F7A); break;
      case 11: __builtin_amdgcn_s_waitcnt(0x0F7B); break;
      case 12: __builtin_amdgcn_s_waitcnt(0x0F7C); break;
      case 13: __builtin_amdgcn_s_waitcnt(0x0F7D); break;
      case 14: __builtin_amdgcn_s_waitcnt(0x0F7E); break;
      case 15: __builtin_amdgcn_s_waitcnt(0x0F7F); break;
      default: __builtin_amdgcn_s_waitcnt(0x4F70); break;  // vmcnt(16)
    }
  };
  static_assert(2 * C::VLOADS <= 16, "wait_vm covers at most 16 DMAs in flight");

  // K operand read addresses (bytes within a slot) for k-step s: lane
  // (m = n, q) reads key row n, dims 32 s + 8 q .. + 8
  int krd[C::NS];
#pragma unroll
  for (int s = 0; s < C::NS; ++s) krd[s] = n * C::ROWB + 16 * kswz<D>(n, 4 * s + q);
  auto read_k = [&](const uint16_t* src, V8 (&kb)[C::NS]) {
#pragma unroll
    for (int s = 0; s < C::NS; ++s) kb[s] = *(const V8*)((const char*)src + krd[s]);
  };

  // V^T operand read addresses (bytes within a slot) for slice s: lane x of
  // its 16-lane group reads ring row 4 q + x/4, dims CW (x%4) + 4 s .. + 3
  int vrd[C::NV];
#pragma unroll
  for (int s = 0; s < C::NV; ++s) {
    const int x = n, R = 4 * q + (x >> 2);
    const int dim0 = C::CW * (x & 3) + 4 * s;
    vrd[s] = R * C::ROWB + 16 * vswz<D>(R, dim0 >> 3) + 2 * (dim0 & 7);
  }

  const float scale = A.scale_log2;
  float m_run = -INFINITY, l_run = 0.f, n_run = 0.f;
  f32x4 oacc[C::NV];
#pragma unroll
  for (int s = 0; s < C::NV; ++s) oacc[s] = f32x4{};

  // This row's scaled score (log2 units) in a 16-key chunk of a band (d =
  // the row's key minus the chunk's first key; no key in the chunk: d < 0 or
  // d >= 16), the same in the row's 4 lanes; -inf when the row has no key
  // there.  has / e: this lane holds the key, at register e (d >> 2 == q
  // only for d in 4 q .. 4 q + 3, an arithmetic shift keeping d < 0 out).
  auto lane_score = [&](const f32x4& sacc, int d, bool& has, int& e) -> float {
    has = (d >> 2) == q;
    e = d & 3;
    const float s01 = (e & 1) ? sacc[1] : sacc[0];
    const float s23 = (e & 1) ? sacc[3] : sacc[2];
    const float s = (e & 2) ? s23 : s01;
    return has ? s * scale : -INFINITY;
  };
  auto pick = [&](const f32x4& sacc, int d, bool& has, int& e) -> float {
    return row4_max(lane_score(sacc, d, has, e));
  };
  // both bands of a pair (one fused 4-lane max)
  auto pick2 = [&](const f32x4& sa, int da, bool& ha, int& ea, float& xa, const f32x4& sb,
                   int db, bool& hb, int& eb, float& xb) {
    xa = lane_score(sa, da, ha, ea);
    xb = lane_score(sb, db, hb, eb);
    row4_max2(xa, xb);
  };
  // Online softmax over two bands' scores xa, xb (one running-max update per
  // pair, so both probabilities share one scale) -> P words (the input type
  // at register e of the lane holding the key, else 0)
  auto pair_softmax = [&](float xa, bool ha, int ea, float xb, bool hb, int eb, uint64_t& pa,
                          uint64_t& pb) {
    const float xm = max_nq(xa, xb);
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float ra = xa - m_use, rb = xb - m_use;
    const float rm = xm - m_use;
    // (a row's first valid key: threshold -inf, and rm = xm there)
    const float thr = m_run == -INFINITY ? -INFINITY : kRescaleSlack;
    const bool grow = rm > thr;
    if (wave_any(grow)) {
      const float delta = grow ? rm : 0.f;
      // rows that do not grow keep alpha = 1 (m_run may still be -inf there)
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
    // O is normalised by the probabilities PV used (rounded to the input type)
    n_run += M::val(b0);
    n_run += M::val(b1);
    pa = (uint64_t)(ha ? b0 : 0u) << (16 * ea);
    pb = (uint64_t)(hb ? b1 : 0u) << (16 * eb);
  };

  auto scores = [&](const V8 (&kb)[C::NS]) {
    f32x4 sacc = M::mfma16(kb[0], qop[0], f32x4{});
#pragma unroll
    for (int s = 1; s < C::NS; ++s) sacc = M::mfma16(kb[s], qop[s], sacc);
    return sacc;
  };

  // V^T operands of two bands from slots va, vb (ds_read_b64_tr_b16); with
  // san, non-finite values become +0 (the rerun of a group whose output met
  // a non-finite value)
  auto read_vt = [&](auto san, const uint16_t* va, const uint16_t* vb, s16x4 (&ta)[C::NV],
                     s16x4 (&tb)[C::NV]) {
#pragma unroll
    for (int s = 0; s < C::NV; ++s) {
      ta[s] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((const char*)va + vrd[s]));
      tb[s] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((const char*)vb + vrd[s]));
    }
    if constexpr (decltype(san)::value) {
#pragma unroll
      for (int s = 0; s < C::NV; ++s) {
        u32x2 a = __builtin_bit_cast(u32x2, ta[s]), c = __builtin_bit_cast(u32x2, tb[s]);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          a[e] = sanitize2<E>(a[e]);
          c[e] = sanitize2<E>(c[e]);
        }
        ta[s] = __builtin_bit_cast(s16x4, a);
        tb[s] = __builtin_bit_cast(s16x4, c);
      }
    }
  };
  // O^T += V^T P^T over two bands' V^T operands ta, tb with P words pa, pb
  // (k-slots 8 q .. 8 q + 3: band a keys 4 q .. 4 q + 3; 8 q + 4 .. 8 q + 7:
  // band b's)
  auto pv = [&](const s16x4 (&ta)[C::NV], const s16x4 (&tb)[C::NV], uint64_t pa,
                uint64_t pb) {
    const u32x4 pq = {(uint32_t)pa, (uint32_t)(pa >> 32), (uint32_t)pb, (uint32_t)(pb >> 32)};
    const V8 pop = __builtin_bit_cast(V8, pq);
#pragma unroll
    for (int s = 0; s < C::NV; ++s) {
      const s16x4 vv[2] = {ta[s], tb[s]};
      oacc[s] = M::mfma16(__builtin_bit_cast(V8, vv), pop, oacc[s]);
    }
  };

  // O^T += V^T P^T reading each 16-dim slice's V^T operands next to its MFMA
  // (D = 256: all slices of both bands at once would hold 64 VGPRs)
  auto pv_sliced = [&](auto san, const uint16_t* va, const uint16_t* vb, uint64_t pa,
                       uint64_t pb) {
    const u32x4 pq = {(uint32_t)pa, (uint32_t)(pa >> 32), (uint32_t)pb, (uint32_t)(pb >> 32)};
    const V8 pop = __builtin_bit_cast(V8, pq);
#pragma unroll
    for (int s = 0; s < C::NV; ++s) {
      s16x4 vv[2] = {
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((const char*)va + vrd[s])),
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((const char*)vb + vrd[s]))};
      if constexpr (decltype(san)::value) {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          u32x2 w = __builtin_bit_cast(u32x2, vv[h2]);
          w[0] = sanitize2<E>(w[0]);
          w[1] = sanitize2<E>(w[1]);
          vv[h2] = __builtin_bit_cast(s16x4, w);
        }
      }
      oacc[s] = M::mfma16(__builtin_bit_cast(V8, vv), pop, oacc[s]);
    }
  };

  // ---- the bands: the main loop over band pairs, then the tail.  san: the
  // rerun with sanitised V operands (see below).
  auto run_bands = [&](auto san) {
    // ---- main loop: band pairs (2 p, 2 p + 1).
    //   VEARLY: wait for the pair's K and V DMAs (the only ones outstanding),
    //   read the K and V^T operands, request the next pair's K and V into the
    //   same slots, then compute from registers.
    //   Otherwise: before the K wait exactly this pair's V DMAs (as many as
    //   load_v issued) may be newer; before the V wait the next pair's K DMAs
    //   (2 VLOADS of them, or with KSKIP as many as load_k issued).
    constexpr int kWaitPair = (0xF70 & ~0xF) | ((2 * C::VLOADS) & 0xF) |
                              (((2 * C::VLOADS) >> 4) << 14);  // vmcnt(2 VLOADS)
    constexpr int kWaitLds = 0xC07F;                           // lgkmcnt(0)
    const int lane_key = 4 * n;  // ds_bpermute byte address of row n in group 0
    {
      const int i0 = __builtin_amdgcn_readlane(info1, 16 * q0);
      const int i1 = __builtin_amdgcn_readlane(info1, 16 * q0 + 1);
      __builtin_amdgcn_s_waitcnt(kWaitLds);  // the slot zeros are in LDS
      load_k(i0, lk0);
      load_k(i1, lk1);
      load_v(i0, lv0);
      load_v(i1, lv1);
    }
    for (int qj = q0; qj < q0 + 4 / S; ++qj) {
      const bool more = qj < q0 + 4 / S - 1;
  #pragma unroll
      for (int rp = 0; rp < 8; ++rp) {
        const int ra = 2 * rp, rb = 2 * rp + 1;
        const int ia = __builtin_amdgcn_readlane(info1, 16 * qj + ra);
        const int ib = __builtin_amdgcn_readlane(info1, 16 * qj + rb);
        // next pair's descriptors (slots 16 qj + ra + 2, + rb + 2: at rp = 7
        // slots 0 and 1 of lane group qj + 1)
        int na = 0, nb = 0;
        if (rp < 7 || more) {
          na = __builtin_amdgcn_readlane(info1, 16 * qj + ra + 2);
          nb = __builtin_amdgcn_readlane(info1, 16 * qj + rb + 2);
        }
        const bool live = (ia | ib) != 0;  // some row of the group uses a band
        const int n_nxt = KSKIP ? n_loads(na) + n_loads(nb) : 2 * C::VLOADS;  // next K DMAs
        V8 kopa[C::NS], kopb[C::NS];
        s16x4 ta[C::NV], tb[C::NV];
        f32x4 sa, sb;
        if constexpr (VEARLY) {
          __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // this pair's K and V are in LDS
          if (live) {
            read_k(ks0, kopa);
            read_k(ks1, kopb);
            read_vt(san, vs0, vs1, ta, tb);
          }
          __builtin_amdgcn_s_waitcnt(kWaitLds);  // slots read: refill them
          load_k(na, lk0);
          load_k(nb, lk1);
          load_v(na, lv0);
          load_v(nb, lv1);
        } else {
          wait_vm(n_loads(ia) + n_loads(ib));  // this pair's K is in LDS
          if (live) {
            read_k(ks0, kopa);
            if constexpr (D == 256) {
              // (one band's K operands at a time: both would hold 64 VGPRs)
              sa = scores(kopa);
              read_k(ks1, kopa);
              sb = scores(kopa);
            } else {
              read_k(ks1, kopb);
            }
          }
          __builtin_amdgcn_s_waitcnt(kWaitLds);  // K slots read: refill them
          load_k(na, lk0);
          load_k(nb, lk1);
        }
        if (live) {
          // the row's key offsets of both bands: bytes ra % 4, rb % 4 of word
          // rp / 2 (the same word for the pair)
          const uint32_t dw =
              (uint32_t)__builtin_amdgcn_ds_bpermute(lane_key + 64 * qj, (int)kd[rp >> 1]);
          const int da = (int)((dw >> (16 * (rp & 1))) & 0xFFu);
          const int db = (int)((dw >> (16 * (rp & 1) + 8)) & 0xFFu);
          if constexpr (VEARLY || D != 256) {
            sa = scores(kopa);
            sb = scores(kopb);
          }
          bool ha, hb;
          int ea, eb;
          float xa, xb;
          pick2(sa, da, ha, ea, xa, sb, db, hb, eb, xb);
          uint64_t pa, pbw;
          pair_softmax(xa, ha, ea, xb, hb, eb, pa, pbw);
          if constexpr (!VEARLY) {
            // this pair's V is in LDS
            if constexpr (KSKIP)
              wait_vm(n_nxt);
            else
              __builtin_amdgcn_s_waitcnt(kWaitPair);
            if constexpr (D != 256) read_vt(san, vs0, vs1, ta, tb);
          }
          if constexpr (!VEARLY && D == 256)
            pv_sliced(san, vs0, vs1, pa, pbw);
          else
            pv(ta, tb, pa, pbw);
        }
        if constexpr (!VEARLY) {
          // this pair's V has landed (and been read): refill the V slots
          if constexpr (KSKIP) {
            wait_vm(n_nxt);
            __builtin_amdgcn_s_waitcnt(kWaitLds);
          } else {
            __builtin_amdgcn_s_waitcnt(kWaitPair & kWaitLds);
          }
          load_v(na, lv0);
          load_v(nb, lv1);
        }
      }
    }

    // ---- tail: keys of bands wider than 16, one 16-key chunk at a time
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    const bool wide = wave_any(((uint32_t)info1 >> 24) > 16u);  // some slot's band
    for (int j = 16 * q0; j < 16 * (q0 + 4 / S) && wide; ++j) {
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
        const int rem = lo + wdt - c0;
        const int ci = c0 | (min(rem, 16) << 24);
        __builtin_amdgcn_s_waitcnt(kWaitLds);  // earlier reads of slots 0 done
        load_k(ci, lk0);
        load_v(ci, lv0);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        V8 kt[C::NS];
        read_k(ks0, kt);
        const f32x4 st = scores(kt);
        bool ht;
        int et;
        const float xt = pick(st, d == 0xFF ? -1 : d - (c0 - lo), ht, et);
        uint64_t pt, pz;
        pair_softmax(xt, ht, et, -INFINITY, false, 0, pt, pz);
        // the second band of the pair contributes p = 0
        if constexpr (D == 256) {
          pv_sliced(san, vs0, vs1, pt, 0ull);
        } else {
          s16x4 ta[C::NV], tb[C::NV];
          read_vt(san, vs0, vs1, ta, tb);
          pv(ta, tb, pt, 0ull);
        }
      }
    }
  };

  run_bands(std::integral_constant<bool, false>{});
  // A group whose outputs met a non-finite value (an Inf or NaN in V, staged
  // with a band, can reach rows that do not list it through 0 * Inf in PV)
  // runs again with the V operands sanitised: rows whose entries bring no
  // non-finite value then get exactly the bits a run without it gives, and
  // the reference's non-finite values go back in below.
  // (with S waves each decides for its own bands: a wave whose sums are
  // finite met no non-finite value, and its sanitised run would give the
  // same bits)
  bool rerun = wave_any(!sum_finite(oacc));
  if (rerun) {
    m_run = -INFINITY;
    l_run = 0.f;
    n_run = 0.f;
#pragma unroll
    for (int s = 0; s < C::NV; ++s) oacc[s] = f32x4{};
    run_bands(std::integral_constant<bool, true>{});
  }
  if constexpr (S > 1) {
    // wave 1 hands its state to wave 0 through its own slots: O^T slices
    // (64 lanes x 16 bytes each, SLOT / 512 per slot) in ks0 and ks1, and
    // (m, l, n, rerun) per lane in vs0
    constexpr int SPS = C::SLOT / 512;
    static_assert(C::NV <= 2 * SPS, "two slots hold the O^T slices");
    f32x4* const ox0 = (f32x4*)(ks0_ + C::SLOT);
    f32x4* const ox1 = (f32x4*)(ks1_ + C::SLOT);
    f32x4* const sx = (f32x4*)(vs0_ + C::SLOT);
    if (wv == 1) {
      __builtin_amdgcn_s_waitcnt(0);  // its DMAs into these slots have landed
#pragma unroll
      for (int s = 0; s < C::NV; ++s) (s < SPS ? ox0 : ox1)[(s % SPS) * 64 + lane] = oacc[s];
      sx[lane] = f32x4{m_run, l_run, n_run, rerun ? 1.f : 0.f};
    }
    __syncthreads();
    if (wv == 1) return;
    const f32x4 st = sx[lane];
    const float m = fmaxf(m_run, st[0]);
    const float a0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m);
    const float a1 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st[0] - m);
    l_run = l_run * a0 + st[1] * a1;
    n_run = n_run * a0 + st[2] * a1;
#pragma unroll
    for (int s = 0; s < C::NV; ++s) {
      const f32x4 o1 = (s < SPS ? ox0 : ox1)[(s % SPS) * 64 + lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) oacc[s][e] = oacc[s][e] * a0 + o1[e] * a1;
    }
    m_run = m;
    rerun = rerun || st[3] != 0.f;
  }

  // ---- epilogue: lane (n, q) holds O^T[dim][row n] for dims CW q .. CW q + CW
  // (slice s, reg e: dim CW q + 4 s + e)
  if (row_ok) {
    const float inv = n_run > 0.f ? 1.f / n_run : 0.f;
    uint16_t* orow = A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)r * A.oss;
#pragma unroll
    for (int t = 0; t < C::NV / 2; ++t) {
      V8 ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ov[e] = (typename M::s)(oacc[2 * t][e] * inv);
        ov[4 + e] = (typename M::s)(oacc[2 * t + 1][e] * inv);
      }
      if (C::CW * q + 8 * t < A.d_real) *(V8*)(orow + C::CW * q + 8 * t) = ov;
    }
    if (A.lse && q == 0) {
      const float lse = l_run > 0.f ? (m_run + __log2f(l_run)) * 0.69314718055994530942f
                                    : -INFINITY;
      A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + r] = lse;
    }
    // after a rerun: the dims where the row's own entries bring an Inf or NaN
    // of V take the reference's value (this lane's dims CW q .. CW q + CW)
    if (rerun) {
      int dim0[C::CW / 4];
#pragma unroll
      for (int g = 0; g < C::CW / 4; ++g) dim0[g] = C::CW * q + 4 * g;
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

template <int D, Elem E, bool POS, int S>
void launch_band_ds(const BandArgs& a, dim3 grid, bool kskip, bool vearly, hipStream_t stream) {
  if (kskip) {
    if (vearly)
      band_fwd_kernel<D, true, true, E, POS, S><<<grid, 64 * S, 0, stream>>>(a);
    else
      band_fwd_kernel<D, true, false, E, POS, S><<<grid, 64 * S, 0, stream>>>(a);
  } else {
    if (vearly)
      band_fwd_kernel<D, false, true, E, POS, S><<<grid, 64 * S, 0, stream>>>(a);
    else
      band_fwd_kernel<D, false, false, E, POS, S><<<grid, 64 * S, 0, stream>>>(a);
  }
}

// Two waves per group where the whole grid fits one round of two-wave
// workgroups (n_groups at most 8 * 40960 / D / 2: 1280 at D = 128, 2560 at
// D = 64), so each group's walk over its 64 bands, the grid's whole time
// there, is split in half
template <int D, Elem E, bool POS>
void launch_band_d(const BandArgs& a, dim3 grid, bool kskip, bool vearly, hipStream_t stream) {
  if (a.n_groups <= 8 * (40960 / D) / 2)
    launch_band_ds<D, E, POS, 2>(a, grid, kskip, vearly, stream);
  else
    launch_band_ds<D, E, POS, 1>(a, grid, kskip, vearly, stream);
}

// D = 256 runs only the late V order: the early one holds both bands' K and
// V^T operands at once (128 VGPRs at D = 256, about 264 in all)
template <Elem E, bool POS>
void launch_band_d256(const BandArgs& a, dim3 grid, bool kskip, hipStream_t stream) {
  if (kskip)
    band_fwd_kernel<256, true, false, E, POS><<<grid, 64, 0, stream>>>(a);
  else
    band_fwd_kernel<256, false, false, E, POS><<<grid, 64, 0, stream>>>(a);
}

// the kernel's D: the head_dim, or the next of 64, 128, 256 above it
template <Elem E>
void launch_band_elem(const BandArgs& a, int head_dim, dim3 grid, bool kskip, bool vearly,
                      hipStream_t stream) {
  if (a.positions) {
    if (head_dim > 128)
      launch_band_d256<E, true>(a, grid, kskip, stream);
    else if (head_dim > 64)
      launch_band_d<128, E, true>(a, grid, kskip, vearly, stream);
    else
      launch_band_d<64, E, true>(a, grid, kskip, vearly, stream);
  } else {
    if (head_dim > 128)
      launch_band_d256<E, false>(a, grid, kskip, stream);
    else if (head_dim > 64)
      launch_band_d<128, E, false>(a, grid, kskip, vearly, stream);
    else
      launch_band_d<64, E, false>(a, grid, kskip, vearly, stream);
  }
}

hipError_t launch_band_fwd(const BandArgs& a, int head_dim, hipStream_t stream) {
  if (a.n_groups <= 0) return hipSuccess;
  // interpolation weight 0 (a sliding window): every group's bands overlap
  // in all but one key per step, so the window kernel stages each key once
  if (window_fwd_applies(a, head_dim)) return launch_window_fwd(a, head_dim, stream);
  dim3 grid((unsigned)(8 * a.per_xcd));
  // The refill order by the entry spacing at the last row, (q_len a + c) / w
  // query rows between one entry's keys and the next's: at B=1 H=8 L=131072
  // D=128 the early V requests were 9-11% faster at spacings 586 and 878
  // (layers 2, 3) and 3-12% slower at 1171 .. 2048 (layers 4-7), where the
  // L2 hit rate fell from 0.73 to 0.64 (layer 4) and HBM misses bound the
  // kernel; at the shapes up to L = 32768 (spacings up to 512) they were
  // faster or within 3.5%.
  // (with positions, the last row sits near kv_len)
  const float last = (float)(a.positions ? a.kv_len : a.q_len);
  const float spacing = (last * a.pc.a + a.pc.c) / (float)a.pc.w;
  const bool vearly = spacing < 1000.0f;
  // Entry rotation.  An XCD keeps 40960 / D waves resident (by LDS: 320 at
  // D = 128, 640 at D = 64, 160 at D = 256).  Where the grid fills many
  // rounds of them, waves finish and are replaced one at a time, a group
  // about every 64 / 320 = 12.8/64 (D = 128) or 6.4/64 (D = 64) of a wave's
  // walk, and a rotation a little ahead of that rate (15/64, 9/64) puts the
  // resident groups on neighbouring entries, whose keys share L2: 15 and 9
  // are the best or within 2% of it at every layer of B=1 H=8 L=131072
  // (12/64 there was 8-11% slower at D = 128 layers 4-7, 17-22% at D = 64).
  // A grid of a few rounds starts each round nearly at once instead, and the
  // same rate spreads a round's groups over all 64 entries, so an XCD's L2
  // must hold the keys of every entry of the resident rows.  Where a head's
  // K and V (4 head_dim bytes per key) exceed the 4 MB L2, a grid of up to
  // four rounds therefore rotates by 3/64 only.  Same box, rotation against
  // none: the last 1024 / 2048 / 4096 rows of B=1 H=32 L=32768 D=128 layer
  // 4 as a chunk (0.8 / 1.6 / 3.2 rounds) 0.108 -> 0.066, 0.179 -> 0.106,
  // 0.271 -> 0.197 ms, layer 7 -7% / -30%, the last 16384 rows of B=1 H=8
  // L=131072 -31% at layer 4 (+3% at layer 7); at 6.4 rounds within +-3%,
  // at 12.8 the rotation 1-9% faster, at 25.6 (the full L=32768 prefill) 9%.
  // At L=8192 (4 MB of K and V per head) none was 1-4% slower at 0.8-3.6
  // rounds.  3/64 against none, same box: the 3.2-round chunks above -2.6%
  // (layer 4) and -5% (layer 7), the L=131072 chunk -9% at layers 4 and 7,
  // B=1 H=2 L=65536 prefill -10%; 0.8-round chunks +1-2%; 2/64 and 4/64
  // each worse at some of these.
  const int dk = head_dim > 128 ? 256 : head_dim > 64 ? 128 : 64;
  BandArgs r = a;
  // Chunks (positions) from interpolation weight 1/2 on keep 3/64 up to
  // eight rounds: their rows all have wide windows, and the late 6144- and
  // 8192-row chunks of L=32768 (4.8 and 6.4 rounds) ran 13-33% faster at
  // layers 4 and 7, the late 32768-row chunks of L=131072 6-34%, early
  // chunks (position 0) within 1%; full prefills at 6.4 rounds up to 15%
  // slower, and late chunks at layer 2 of L=131072 18-36% slower.
  const int max_rounds = a.positions && a.pc.a >= 0.5f ? 8 : 4;
  r.rot_rate = band_rotation(a.n_groups, 40960 / dk, (int64_t)a.kv_len * 4 * a.d_real,
                             dk == 128 ? 15 : 9, 3, max_rounds);
  // K DMA skipping: with the late V order from interpolation weight 1/2 on
  // (measured at B=1, H=32, L=32768, D=128, w=64 over 8 layers: 1-7% faster
  // at weights 4/7 .. 1, even at 3/7, 3-4% slower at 1/7 and 2/7, where
  // nearly every band is 16 keys wide and the run-time waits cost more than
  // the DMAs saved); with the early V order (one vmcnt(0) wait per pair,
  // whatever the count) always: 2-5% faster at weights 2/7 and 3/7 of
  // L=8192 .. 131072, within 1% at 1/7
  const bool kskip = a.pc.a >= 0.5f || vearly;
  if (a.elem == (int)Elem::f16)
    launch_band_elem<Elem::f16>(r, head_dim, grid, kskip, vearly, stream);
  else
    launch_band_elem<Elem::bf16>(r, head_dim, grid, kskip, vearly, stream);
  return hipGetLastError();
}

}  // namespace esa
