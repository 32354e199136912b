// Block-sparse flash-attention backward over the elastic pattern (gfx950).
//
// Replaces the backward branch of the reference's per-token Triton kernel
// (elastic_sparse_attention.py:168-233, launched from :299-339), which
// recomputes each query row's probabilities and scatters dK and dV with float
// atomics.  Here every gradient is accumulated by exactly one workgroup, in a
// fixed order, so the result is deterministic:
//
//   prep_kernel      delta = rowsum(dO * O) and lse2 = lse * log2(e) per row
//   tile_mask_kernel for every active tile of the layout, the key-major mask:
//                    per 32-row query sub-block and key, the 32 row bits
//                    (each row's elastic index walk, then a 32x32 bit
//                    transpose by lane butterflies)
//   dkdv_kernel      one workgroup per (batch, kv head, 128-key block): the
//                    block's K and V rows stay in registers; it visits every
//                    (head, query block) tile that lists the key block (the
//                    transposed layout), recomputes S = Q K^T and P, and
//                    accumulates dV^T += dO^T P and dK^T += Q^T dS
//   dq_kernel        one workgroup per (batch, head, 128-row query block),
//                    over the block's active tiles like the forward:
//                    dQ^T += K^T dS^T
//
// with P = exp(S * scale - lse) on valid keys, dS = P * (dO V^T - delta),
// dQ = scale * dS K and dK = scale * dS^T Q (:191-228).  A 32 x 32 block whose
// rows have no valid key contributes nothing and is skipped.  Operand layouts
// and LDS staging follow the forward kernel (buffer_load ... lds, XOR-swizzled
// rows, one 64-row stage ahead); a buffer read with both the 16-byte row
// pattern and the ds_read_b64_tr_b16 pattern uses the K swizzle, which is
// conflict-free for both.
#include "esa_tile.hpp"

namespace esa {

namespace {

template <int D>
struct BwdCfg {
  static constexpr int HALF = 64;                 // rows per stage
  static constexpr int CPR = D / 8;               // 16-byte chunks per row
  static constexpr int STAGE = HALF * D;          // elements per stage buffer
  static constexpr int LOADS = HALF * CPR / 256;  // 16-byte loads per lane per matrix per stage
  static constexpr int NS = D / 16;               // k-steps over d
  static constexpr int ND = D / 32;               // 32-wide d blocks
};

__device__ __forceinline__ void load_lds4(__amdgpu_buffer_rsrc_t rsrc, float* dst, int voffset,
                                          int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)dst, 4, voffset, soffset, 0, 0);
}

// 32 x 32 bit transpose across the lanes of each 32-lane half: on entry lane
// r holds row r; on exit lane k holds column k (bit r = row r's bit k).
__device__ __forceinline__ uint32_t transpose32(uint32_t x, int lane) {
  const uint32_t masks[5] = {0x0000FFFFu, 0x00FF00FFu, 0x0F0F0F0Fu, 0x33333333u, 0x55555555u};
#pragma unroll
  for (int step = 0; step < 5; ++step) {
    const int j = 16 >> step;
    const uint32_t m = masks[step];
    const uint32_t y = (uint32_t)__shfl_xor((int)x, j, 32);
    x = (lane & j) ? ((x & ~m) | ((y & ~m) >> j)) : ((x & m) | ((y & m) << j));
  }
  return x;
}

}  // namespace

// ---------------------------------------------------------------------------
// delta and lse in log2 units, one 16-lane group per query row, PREP_ROWS
// rows per workgroup (four 16-row passes, every pass's O and dO loads issued
// before the first sum: a 16-row workgroup per launch slot left the kernel
// bound by load latency, 3 TB/s at B=8 H=16 L=4096 D=64).  Each row's sum
// runs in the same order as before and as the band dQ kernel's (lane g adds
// its D/16 products in turn, then xor shuffles 8, 4, 2, 1).  heads_fast: the
// grid's fastest axis is the head (blockIdx.x = h, blockIdx.y = row block),
// so where O's heads lie inside a row ([B, L, H, D], the forward's output)
// neighbouring blocks read neighbouring bytes; otherwise the axes swap.
constexpr int PREP_ROWS = 64;

template <int D, Elem E>
__global__ __launch_bounds__(256) void prep_kernel(BwdArgs A, float* lse2, int heads_fast) {
  using M = MmaT<E>;
  constexpr int PER = D / 16;  // elements per lane
  constexpr int PASSES = PREP_ROWS / 16;
  // PER 16-bit elements as one load
  typedef uint32_t chunk_t __attribute__((ext_vector_type(PER / 2)));
  const int rb = heads_fast ? blockIdx.y : blockIdx.x;
  const int h = heads_fast ? blockIdx.x : blockIdx.y, b = blockIdx.z;
  const int g = threadIdx.x & 15;
  if (A.split_parts > 1 && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0)
    for (int i = threadIdx.x; i < A.n_bkv * A.split_blocks; i += 256)
      A.part_cnt[i] = 0;  // split arrivals
  const uint16_t* ob = A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + g * PER;
  const uint16_t* db = A.dout + (int64_t)b * A.dosb + (int64_t)h * A.dosh + g * PER;
  chunk_t ov[PASSES], dv[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int row = rb * PREP_ROWS + p * 16 + (threadIdx.x >> 4);
    ov[p] = dv[p] = chunk_t{};
    if (row < A.q_len) {
      ov[p] = *(const chunk_t*)(ob + (int64_t)row * A.oss);
      dv[p] = *(const chunk_t*)(db + (int64_t)row * A.doss);
    }
  }
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int row = rb * PREP_ROWS + p * 16 + (threadIdx.x >> 4);
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const uint32_t ow = ov[p][e >> 1], dw = dv[p][e >> 1];
      acc += M::val(e & 1 ? ow >> 16 : ow & 0xffffu) * M::val(e & 1 ? dw >> 16 : dw & 0xffffu);
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 16);
    if (row < A.q_len && g == 0) {
      const int64_t at = ((int64_t)b * A.H + h) * A.qpad + row;
      A.delta[at] = acc;
      // kept finite: masked scores enter as -inf, and -inf - (-inf) would be NaN
      lse2[at] = fmaxf(A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + row] * 1.4426950408889634f,
                       -3.0e38f);
    }
  }
}

// ---------------------------------------------------------------------------
// Key-major masks of every active tile: mask_t[t][qs][k] bit r = row
// 32 qs + r of the tile's query block has key k0 + k among its valid entries.
__global__ __launch_bounds__(256) void tile_mask_kernel(PatternConsts pc, const int32_t* row_ptr,
                                                        const int32_t* col_idx, int nqb, int nq,
                                                        int q_len, uint32_t* __restrict__ mask_t) {
  const int qb = blockIdx.x, h = blockIdx.y;
  if (qb >= nq) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31;
  const int i = qb * 128 + wave * 32 + l32;
  RowWalker walk;
  walk.init(pc, h, i, i < q_len);
  const int64_t r = (int64_t)h * nqb + qb;
  const int t0 = row_ptr[r], t1 = row_ptr[r + 1];
  for (int t = t0; t < t1; ++t) {
    uint32_t mb[4];
    walk.tile(col_idx[t] * 128, mb);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t col = transpose32(mb[q], l32);
      if (lane < 32) mask_t[(int64_t)t * 512 + wave * 128 + q * 32 + l32] = col;
    }
  }
}

// ---------------------------------------------------------------------------
// dK, dV of one (batch, kv head, 128-key block): 8 waves, one workgroup per
// CU at D = 128.  The block's K and V rows are staged into LDS once (64 KB at
// D = 128) and read as MFMA operands from there, so each wave keeps only its
// dK^T and dV^T accumulators resident and two waves share each SIMD.  At
// D = 64 the workgroup takes 66.5 KB of LDS and the launch bound holds it to
// 128 VGPRs (four spilled: one 8-byte reload per key-block tile), so two
// workgroups share a CU: 7-12% faster than one at 133 VGPRs (B=8 H=16 L=4096 and B=4 H=32
// L=4096, layers 0-5), the same bits.  Wave w owns
// keys 32 (w % 4) .. + 31 of the block and the 32-row half w / 4 of every
// 64-row Q / dO stage; the two halves' partial sums are added through LDS at
// the end, in a fixed order.
template <int D, Elem E>
__global__ __launch_bounds__(512, D == 64 ? 4 : 1) void dkdv_kernel(BwdArgs A, const float* lse2) {
  using M = MmaT<E>;
  using V8 = typename M::v8;
  using C = BwdCfg<D>;
  constexpr int KB = 128;                           // keys per item
  constexpr int KLOADS = KB * C::CPR / 512;         // 16-byte loads per lane per matrix (block)
  constexpr int QLOADS = C::HALF * C::CPR / 512;    // 16-byte loads per lane per matrix (stage)
  static_assert(KLOADS >= 1 && QLOADS >= 1, "at least one load per lane");
  // K rows at kv_blk[0, KB D), V rows at kv_blk[KB D, 2 KB D); the same
  // space holds the partial-sum exchange at the end
  __shared__ __attribute__((aligned(1024))) uint16_t kv_blk[2 * KB * D];
  __shared__ __attribute__((aligned(1024))) uint16_t q_st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t o_st0[C::STAGE];  // dO rows
  __shared__ __attribute__((aligned(1024))) uint16_t q_st1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t o_st1[C::STAGE];
  __shared__ __attribute__((aligned(256))) float l_st0[C::HALF], d_st0[C::HALF];
  __shared__ __attribute__((aligned(256))) float l_st1[C::HALF], d_st1[C::HALF];
  const cptr_i32 kv_items = (cptr_i32)A.kv_items;
  const cptr_i32 kv_ptr = (cptr_i32)A.kv_ptr;
  const cptr_i32 kv_tiles = (cptr_i32)A.kv_tiles;
  const cptr_i32 tile_row = (cptr_i32)A.tile_row;

  const int item = kv_items[blockIdx.x];
  if (item < 0 || item >= A.B * A.Hkv * A.nkb) return;
  const int kb = item % A.nkb;
  const int bkv = item / A.nkb;
  const int kvh = bkv % A.Hkv, b = bkv / A.Hkv;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kw = wave & 3, qh = wave >> 2;  // key sub-block, query half
  const int hf = lane >> 5, l32 = lane & 31, g4 = lane >> 4, lam = lane & 15;
  const int key = kb * KB + kw * 32 + l32;
  const bool key_ok = key < A.kv_len;

  // ---- the key block's K and V rows -> LDS (rows past kv_len read as zeros)
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh), (short)0,
      (int)((int64_t)A.kv_len * A.kss * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh), (short)0,
      (int)((int64_t)A.kv_len * A.vss * 2), 0x00020000);
#pragma unroll
  for (int j = 0; j < KLOADS; ++j) {
    const int slot = (KLOADS * wave + j) * 64 + lane;
    const int row = slot / C::CPR, pc = slot % C::CPR;
    const int chunk = 8 * (pc ^ swz_k<D>(row));
    load_lds16(krs, kv_blk + (KLOADS * wave + j) * 512, (row * (int)A.kss + chunk) * 2,
               kb * KB * (int)A.kss * 2);
    load_lds16(vrs, kv_blk + KB * D + (KLOADS * wave + j) * 512, (row * (int)A.vss + chunk) * 2,
               kb * KB * (int)A.vss * 2);
  }

  f32x16 dkacc[C::ND], dvacc[C::ND];
#pragma unroll
  for (int d = 0; d < C::ND; ++d) {
    dkacc[d] = f32x16{};
    dvacc[d] = f32x16{};
  }

  // staging: Q and dO rows of one 64-row half of a (head, query block) tile
  int qoff[QLOADS], ooff[QLOADS];
#pragma unroll
  for (int j = 0; j < QLOADS; ++j) {
    const int slot = (QLOADS * wave + j) * 64 + lane;
    const int row = slot / C::CPR, pc = slot % C::CPR;
    qoff[j] = (row * (int)A.qss + 8 * (pc ^ swz_k<D>(row))) * 2;
    ooff[j] = (row * (int)A.doss + 8 * (pc ^ swz_k<D>(row))) * 2;
  }
  const int e0 = kv_ptr[kvh * A.nkb + kb], e1 = kv_ptr[kvh * A.nkb + kb + 1];
  auto issue = [&](int e, int hh, uint16_t* qd, uint16_t* od, float* ld, float* dd) {
    const int t = kv_tiles[e];
    const int hq = tile_row[t];
    const int h = hq / A.nqb, qb = hq % A.nqb;
    const int r0 = qb * 128 + C::HALF * hh;
    const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh), (short)0,
        (int)((int64_t)A.q_len * A.qss * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(A.dout + (int64_t)b * A.dosb + (int64_t)h * A.dosh), (short)0,
        (int)((int64_t)A.q_len * A.doss * 2), 0x00020000);
    const int qs_ = r0 * (int)A.qss * 2, os_ = r0 * (int)A.doss * 2;
#pragma unroll
    for (int j = 0; j < QLOADS; ++j) {
      load_lds16(qrs, qd + (QLOADS * wave + j) * 512, qoff[j], qs_);
      load_lds16(ors, od + (QLOADS * wave + j) * 512, ooff[j], os_);
    }
    if (wave < 2) {
      const float* src = (wave == 0 ? lse2 : A.delta) + ((int64_t)b * A.H + h) * A.qpad;
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)src, (short)0, A.q_len * 4, 0x00020000);
      load_lds4(rs, wave == 0 ? ld : dd, lane * 4, r0 * 4);
    }
  };

  // LDS read addresses (elements): 16-byte row reads (rows 32 s2 + l32 of a
  // stage, rows 32 kw + l32 of the key block; chunk 2 s + hf) and transposed
  // reads (rows 4 hf + lam / 4 + 16 u (+ 8), column 32 d + 16 (g4 & 1) +
  // 4 (lam & 3)), all under the K swizzle
  //   chunk (2 s + hf) ^ x = 2 (s ^ (x >> 1)) + (hf ^ (x & 1)), and the row
  //   base leaves bits 4.. of the element offset free below the row, so
  //   raddr(s) = rb ^ 16 s and, likewise, taddr(d) = tb ^ 32 d (one register
  //   each instead of one per s or d)
  const int rx = swz_k<D>(l32);
  const int rb = (l32 * D + 8 * (hf ^ (rx & 1))) | (16 * (rx >> 1));
  int tb0, tb8;
  {
    const int tr = 4 * hf + (lam >> 2);
    const int low = 2 * (g4 & 1) + ((lam >> 1) & 1);  // (col >> 3) & 3
    const int x0 = swz_k<D>(tr), x8 = swz_k<D>(tr + 8);
    tb0 = (tr * D + 8 * (low ^ (x0 & 3)) + 4 * (lam & 1)) | (32 * (x0 >> 2));
    tb8 = ((tr + 8) * D + 8 * (low ^ (x8 & 3)) + 4 * (lam & 1)) | (32 * (x8 >> 2));
  }

  const uint16_t* kblk = kv_blk + kw * 32 * D;       // this wave's K rows
  const uint16_t* vblk = kv_blk + (KB + kw * 32) * D;  // and V rows
  const float scale2 = A.scale_log2;

  // this wave's 32-row query half of a stage held in (qb_, ob_, lb_, db_)
  auto sub = [&](const uint16_t* qb_, const uint16_t* ob_, const float* lb_, const float* db_,
                 uint32_t mw) {
    // rows 8 (r / 4) + 4 hf + r % 4 of the half, key l32 of the wave
    if (!wave_any(mw != 0u)) return;
    // the address bases pass through an empty asm, so the compiler forms
    // each XORed address where it is used instead of keeping one register
    // per address live across the loop
    int rbl = rb, t0l = tb0, t8l = tb8;
    asm volatile("" : "+v"(rbl), "+v"(t0l), "+v"(t8l));
    auto raddr = [&](int s) { return rbl ^ (16 * s); };
    auto taddr0 = [&](int d) { return t0l ^ (32 * d); };
    auto taddr8 = [&](int d) { return t8l ^ (32 * d); };
    const int qrow = 32 * qh * D;
    // the mask enters as S's initial value (0 or -inf), so p = exp2(...) is 0
    // for a masked entry without a select
    f32x16 sacc, dp = f32x16{};
    mask_init<0>(sacc, ~(mw >> (4 * hf)));
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
      const V8 qa = *(const V8*)(qb_ + raddr(s) + qrow);
      const V8 kbv = *(const V8*)(kblk + raddr(s));
      sacc = M::mfma32(qa, kbv, sacc);
    }
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
      const V8 oa = *(const V8*)(ob_ + raddr(s) + qrow);
      const V8 vbv = *(const V8*)(vblk + raddr(s));
      dp = M::mfma32(oa, vbv, dp);
    }
    uint32_t pw[8], sw[8];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int rbase = 32 * qh + 8 * g + 4 * hf;
      const f32x4 lv = *(const f32x4*)(lb_ + rbase);
      const f32x4 dv = *(const f32x4*)(db_ + rbase);
      float p[4], ds[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[4 * g + e], scale2, -lv[e]));
        ds[e] = p[e] * (dp[4 * g + e] - dv[e]);
      }
      pw[2 * g] = M::pack2(p[0], p[1]);
      pw[2 * g + 1] = M::pack2(p[2], p[3]);
      sw[2 * g] = M::pack2(ds[0], ds[1]);
      sw[2 * g + 1] = M::pack2(ds[2], ds[3]);
    }
    // dV^T += dO^T P and dK^T += Q^T dS (query permutation shared by A and B)
#pragma unroll
    for (int d = 0; d < C::ND; ++d) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ro = (32 * qh + 16 * u) * D;
        const s16x4 o1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(ob_ + taddr0(d) + ro));
        const s16x4 o2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(ob_ + taddr8(d) + ro));
        const s16x4 q1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(qb_ + taddr0(d) + ro));
        const s16x4 q2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(qb_ + taddr8(d) + ro));
        const s16x4 oo[2] = {o1, o2}, qq[2] = {q1, q2};
        const u32x4 pq = {pw[4 * u], pw[4 * u + 1], pw[4 * u + 2], pw[4 * u + 3]};
        const u32x4 sq = {sw[4 * u], sw[4 * u + 1], sw[4 * u + 2], sw[4 * u + 3]};
        dvacc[d] = M::mfma32(__builtin_bit_cast(V8, oo), __builtin_bit_cast(V8, pq), dvacc[d]);
        dkacc[d] = M::mfma32(__builtin_bit_cast(V8, qq), __builtin_bit_cast(V8, sq), dkacc[d]);
      }
    }
  };

  const uint32_t* mt = A.mask_t;
  if (e0 < e1) issue(e0, 0, q_st0, o_st0, l_st0, d_st0);
  for (int e = e0; e < e1; ++e) {
    const int64_t t = kv_tiles[e];
    // this wave's query sub-blocks of the tile: qh (stage 0) and 2 + qh (stage 1)
    const uint32_t* tm = mt + t * 512 + kw * 32 + l32;
    const uint32_t ma = tm[qh * 128], mb = tm[(2 + qh) * 128];

    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    issue(e, 1, q_st1, o_st1, l_st1, d_st1);
    sub(q_st0, o_st0, l_st0, d_st0, ma);

    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (e + 1 < e1) issue(e + 1, 0, q_st0, o_st0, l_st0, d_st0);
    sub(q_st1, o_st1, l_st1, d_st1, mb);
  }

  // ---- the second query half's partial sums -> the first half's waves,
  // through the K/V block space (4 key sub-blocks x 16 regs x 64 lanes)
  f32x4* red = (f32x4*)kv_blk;
  auto exchange = [&](f32x16 (&acc)[C::ND]) {
    __syncthreads();
    if (qh == 1) {
#pragma unroll
      for (int d = 0; d < C::ND; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 v4 = {acc[d][4 * g], acc[d][4 * g + 1], acc[d][4 * g + 2], acc[d][4 * g + 3]};
          red[((kw * C::ND + d) * 4 + g) * 64 + lane] = v4;
        }
    }
    __syncthreads();
    if (qh == 0) {
#pragma unroll
      for (int d = 0; d < C::ND; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 v4 = red[((kw * C::ND + d) * 4 + g) * 64 + lane];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[d][4 * g + e] += v4[e];
        }
    }
  };
  exchange(dvacc);
  exchange(dkacc);

  // the non-finite flags of this wave's two 16-key blocks (bwd_fix_kernel
  // recomputes flagged blocks)
  if (qh == 0) {
    const bool bad = wave_any(!sum_finite(dkacc) || !sum_finite(dvacc));
    const int blk = (kb * KB + kw * 32) / 16;
    if (lane < 2 && blk + lane < A.nkb16)
      A.flags[A.n_qflags + (int64_t)bkv * A.nkb16 + blk + lane] = bad ? 1 : 0;
  }
  // dK = scale * (dK^T)^T, dV = (dV^T)^T: lane holds key l32, d = 32 d' +
  // 8 (r / 4) + 4 hf + r % 4
  if (qh == 0 && key_ok) {
    uint16_t* dkr = A.dk + (int64_t)b * A.dksb + (int64_t)kvh * A.dksh + (int64_t)key * A.dkss;
    uint16_t* dvr = A.dv + (int64_t)b * A.dvsb + (int64_t)kvh * A.dvsh + (int64_t)key * A.dvss;
#pragma unroll
    for (int d = 0; d < C::ND; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        typename M::v4 kv4, vv4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kv4[e] = (typename M::s)(dkacc[d][4 * g + e] * A.sm_scale);
          vv4[e] = (typename M::s)(dvacc[d][4 * g + e]);
        }
        *(typename M::v4*)(dkr + 32 * d + 8 * g + 4 * hf) = kv4;
        *(typename M::v4*)(dvr + 32 * d + 8 * g + 4 * hf) = vv4;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// PRE: each row's valid keys per tile come from A.qmask (written once per
// layout by stage_mask_kernel, the bits the walk computes), one 16-byte load
// per tile, issued a tile ahead, in place of the index walk.
template <int D, Elem E, bool PRE>
__global__ __launch_bounds__(256, 2) void dq_kernel(BwdArgs A, const float* lse2) {
  using M = MmaT<E>;
  using V8 = typename M::v8;
  using C = BwdCfg<D>;
  __shared__ __attribute__((aligned(1024))) uint16_t k_st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t v_st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t k_st1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t v_st1[C::STAGE];
  const cptr_i32 items = (cptr_i32)A.q_items;
  const cptr_i32 row_ptr = (cptr_i32)A.row_ptr;
  const cptr_i32 col_idx = (cptr_i32)A.col_idx;

  const int item = items[blockIdx.x];
  if (item < 0 || item >= A.B * A.H * A.nqb) return;
  const int qb = item % A.nqb;
  if (qb >= A.nq) return;
  const int bh = item / A.nqb;
  const int h = bh % A.H, b = bh / A.H;
  const int kvh = h / A.groups;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hf = lane >> 5, l32 = lane & 31, g4 = lane >> 4, lam = lane & 15;
  const int i = qb * 128 + wave * 32 + l32;
  const bool row_ok = i < A.q_len;

  // Q and dO of this lane's row as B operands (8 consecutive d per lane)
  V8 qop[C::NS], oop[C::NS];
  {
    const uint16_t* qr = A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)i * A.qss;
    const uint16_t* dr = A.dout + (int64_t)b * A.dosb + (int64_t)h * A.dosh + (int64_t)i * A.doss;
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
      u32x4 qraw = {0u, 0u, 0u, 0u}, draw = {0u, 0u, 0u, 0u};
      if (row_ok) {
        qraw = *(const u32x4*)(qr + 16 * s + 8 * hf);
        draw = *(const u32x4*)(dr + 16 * s + 8 * hf);
      }
      qop[s] = __builtin_bit_cast(V8, qraw);
      oop[s] = __builtin_bit_cast(V8, draw);
    }
  }
  float l2 = 0.f, dl = 0.f;
  if (row_ok) {
    const int64_t at = ((int64_t)b * A.H + h) * A.qpad + i;
    l2 = lse2[at];
    dl = A.delta[at];
  }
  RowWalker walk;
  if (!PRE) walk.init(A.pc, h, i, row_ok);
  f32x16 dqacc[C::ND];
#pragma unroll
  for (int d = 0; d < C::ND; ++d) dqacc[d] = f32x16{};

  const int64_t lrow = (int64_t)h * A.nqb + qb;
  const int t0 = row_ptr[lrow], t1 = row_ptr[lrow + 1];
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh), (short)0,
      (int)((int64_t)A.kv_len * A.kss * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh), (short)0,
      (int)((int64_t)A.kv_len * A.vss * 2), 0x00020000);
  int koff[C::LOADS], voff[C::LOADS];
#pragma unroll
  for (int j = 0; j < C::LOADS; ++j) {
    const int slot = (C::LOADS * wave + j) * 64 + lane;
    const int row = slot / C::CPR, pc = slot % C::CPR;
    koff[j] = (row * (int)A.kss + 8 * (pc ^ swz_k<D>(row))) * 2;
    voff[j] = (row * (int)A.vss + 8 * (pc ^ swz_k<D>(row))) * 2;
  }
  auto issue = [&](int kt, int hh, uint16_t* kd, uint16_t* vd) {
    const int key0 = col_idx[kt] * 128 + C::HALF * hh;
    const int ks = key0 * (int)A.kss * 2, vs = key0 * (int)A.vss * 2;
#pragma unroll
    for (int j = 0; j < C::LOADS; ++j) {
      load_lds16(krs, kd + (C::LOADS * wave + j) * 512, koff[j], ks);
      load_lds16(vrs, vd + (C::LOADS * wave + j) * 512, voff[j], vs);
    }
  };
  int raddr[C::NS], taddr0[C::ND], taddr8[C::ND];
#pragma unroll
  for (int s = 0; s < C::NS; ++s) raddr[s] = l32 * D + 8 * ((2 * s + hf) ^ swz_k<D>(l32));
  {
    const int tr = 4 * hf + (lam >> 2);
#pragma unroll
    for (int d = 0; d < C::ND; ++d) {
      const int col = 32 * d + 16 * (g4 & 1) + 4 * (lam & 3);
      taddr0[d] = tr * D + 8 * ((col >> 3) ^ swz_k<D>(tr)) + (col & 7);
      taddr8[d] = (tr + 8) * D + 8 * ((col >> 3) ^ swz_k<D>(tr + 8)) + (col & 7);
    }
  }
  const float scale2 = A.scale_log2;

  // one 32-key block kbl of a stage held in (Kb, Vb); mbits: this row's bits
  auto block = [&](const uint16_t* Kb, const uint16_t* Vb, int kbl, uint32_t mbits) {
    // lane half hf holds keys 8 (r / 4) + 4 hf + r % 4 of the block
    const uint32_t mk = mbits >> (4 * hf);
    if (!wave_any(mk != 0u)) return;
    V8 ra[C::NS];
#pragma unroll
    for (int s = 0; s < C::NS; ++s) ra[s] = *(const V8*)(Kb + raddr[s] + 32 * kbl * D);
    // the mask enters as S's initial value (0 or -inf): p = 0 without a select
    f32x16 sacc;
    mask_init<0>(sacc, ~mk);
#pragma unroll
    for (int s = 0; s < C::NS; ++s) sacc = M::mfma32(ra[s], qop[s], sacc);
#pragma unroll
    for (int s = 0; s < C::NS; ++s) ra[s] = *(const V8*)(Vb + raddr[s] + 32 * kbl * D);
    f32x16 dp = f32x16{};
#pragma unroll
    for (int s = 0; s < C::NS; ++s) dp = M::mfma32(ra[s], oop[s], dp);
    uint32_t sw[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float ds[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int r = 2 * q + e;
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], scale2, -l2));
        ds[e] = p * (dp[r] - dl);
      }
      sw[q] = M::pack2(ds[0], ds[1]);
    }
#pragma unroll
    for (int d = 0; d < C::ND; ++d) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ro = (32 * kbl + 16 * u) * D;
        const s16x4 k1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(Kb + taddr0[d] + ro));
        const s16x4 k2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(Kb + taddr8[d] + ro));
        const s16x4 kk[2] = {k1, k2};
        const u32x4 sq = {sw[4 * u], sw[4 * u + 1], sw[4 * u + 2], sw[4 * u + 3]};
        dqacc[d] = M::mfma32(__builtin_bit_cast(V8, kk), __builtin_bit_cast(V8, sq), dqacc[d]);
      }
    }
  };

  // row r's words of tile t at qmask[(t * 128 + r) * 4 ..]
  const uint32_t* qm = PRE ? A.qmask + (wave * 32 + l32) * 4 : nullptr;
  auto load_masks = [&](int t, uint32_t (&m)[4]) {
    u32x4 w = {0u, 0u, 0u, 0u};
    if (row_ok) w = *(const u32x4*)(qm + (int64_t)t * 512);
#pragma unroll
    for (int q = 0; q < 4; ++q) m[q] = w[q];
  };
  uint32_t mnext[4] = {0u, 0u, 0u, 0u};
  if (PRE && t0 < t1) load_masks(t0, mnext);
  if (t0 < t1) issue(t0, 0, k_st0, v_st0);
  for (int t = t0; t < t1; ++t) {
    uint32_t mb[4];
    if (PRE) {
#pragma unroll
      for (int q = 0; q < 4; ++q) mb[q] = mnext[q];
    } else {
      walk.tile(col_idx[t] * 128, mb);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    issue(t, 1, k_st1, v_st1);
    if (PRE && t + 1 < t1) load_masks(t + 1, mnext);
    block(k_st0, v_st0, 0, mb[0]);
    block(k_st0, v_st0, 1, mb[1]);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (t + 1 < t1) issue(t + 1, 0, k_st0, v_st0);
    block(k_st1, v_st1, 0, mb[2]);
    block(k_st1, v_st1, 1, mb[3]);
  }

  // the non-finite flags of this wave's two 16-row groups (bwd_fix_kernel
  // recomputes flagged groups)
  {
    const bool bad = wave_any(!sum_finite(dqacc));
    const int grp = (qb * 128 + wave * 32) / 16;
    if (lane < 2 && grp + lane < A.ng)
      A.flags[((int64_t)b * A.H + h) * A.ng + grp + lane] = bad ? 1 : 0;
  }
  // dQ = scale * (dQ^T)^T: lane holds row i, d = 32 d' + 8 (r / 4) + 4 hf + r % 4
  if (row_ok) {
    uint16_t* dqr = A.dq + (int64_t)b * A.dqsb + (int64_t)h * A.dqsh + (int64_t)i * A.dqss;
#pragma unroll
    for (int d = 0; d < C::ND; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        typename M::v4 q4;
#pragma unroll
        for (int e = 0; e < 4; ++e) q4[e] = (typename M::s)(dqacc[d][4 * g + e] * A.sm_scale);
        *(typename M::v4*)(dqr + 32 * d + 8 * g + 4 * hf) = q4;
      }
    }
  }
}

hipError_t launch_tile_masks(const PatternConsts& pc, const int32_t* row_ptr, const int32_t* col_idx,
                             int nqb, int q_len, uint32_t* mask_t, hipStream_t stream) {
  const int nq = (q_len + 127) / 128;
  if (nq <= 0) return hipSuccess;
  tile_mask_kernel<<<dim3((unsigned)nq, (unsigned)pc.H), 256, 0, stream>>>(pc, row_ptr, col_idx,
                                                                           nqb, nq, q_len, mask_t);
  return hipGetLastError();
}

template <Elem E>
static hipError_t launch_tile_bwd_elem(const BwdArgs& a, int head_dim, int64_t num_q_items,
                                       int64_t num_kv_items, hipStream_t stream) {
  // lse in log2 units goes in the second half of the delta workspace
  float* lse2 = a.delta + (int64_t)a.B * a.H * a.qpad;
  if (num_q_items < 0 && num_kv_items < 0) {
    // both halves band-gathered: the dQ kernel forms delta / lse2 (and clears
    // the split counters) on its way, then dK / dV reads them
    hipError_t e0 = launch_band_dq(a, head_dim, lse2, true, stream);
    if (e0 != hipSuccess) return e0;
    e0 = launch_band_dkdv(a, head_dim, lse2, stream);
    if (e0 != hipSuccess) return e0;
    return launch_bwd_fix(a, head_dim, stream);
  }
  const unsigned n_rb = (unsigned)((a.q_len + PREP_ROWS - 1) / PREP_ROWS);
  // heads fastest where O interleaves heads within a row and the row blocks
  // fit the grid's second axis (65535)
  const int heads_fast = a.osh < a.oss && n_rb <= 65535u;
  const dim3 pg = heads_fast ? dim3((unsigned)a.H, n_rb, (unsigned)a.B)
                             : dim3(n_rb, (unsigned)a.H, (unsigned)a.B);
  if (head_dim == 128)
    prep_kernel<128, E><<<pg, 256, 0, stream>>>(a, lse2, heads_fast);
  else
    prep_kernel<64, E><<<pg, 256, 0, stream>>>(a, lse2, heads_fast);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (num_kv_items < 0) {  // no work list: band-gathered dK / dV
    e = launch_band_dkdv(a, head_dim, lse2, stream);
    if (e != hipSuccess) return e;
  } else if (num_kv_items > 0) {
    if (head_dim == 128)
      dkdv_kernel<128, E><<<dim3((unsigned)num_kv_items), 512, 0, stream>>>(a, lse2);
    else
      dkdv_kernel<64, E><<<dim3((unsigned)num_kv_items), 512, 0, stream>>>(a, lse2);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (num_q_items < 0) {  // no work list
    e = launch_band_dq(a, head_dim, lse2, false, stream);
    if (e != hipSuccess) return e;
    return launch_bwd_fix(a, head_dim, stream);
  }
  if (num_q_items > 0) {
    const dim3 grid((unsigned)num_q_items);
    if (head_dim == 128 && a.qmask)
      dq_kernel<128, E, true><<<grid, 256, 0, stream>>>(a, lse2);
    else if (head_dim == 128)
      dq_kernel<128, E, false><<<grid, 256, 0, stream>>>(a, lse2);
    else if (a.qmask)
      dq_kernel<64, E, true><<<grid, 256, 0, stream>>>(a, lse2);
    else
      dq_kernel<64, E, false><<<grid, 256, 0, stream>>>(a, lse2);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return launch_bwd_fix(a, head_dim, stream);
}

hipError_t launch_tile_bwd(const BwdArgs& a, int head_dim, int64_t num_q_items,
                           int64_t num_kv_items, hipStream_t stream) {
  if (a.q_len <= 0 || a.B <= 0) return hipSuccess;
  if (a.elem == (int)Elem::f16)
    return launch_tile_bwd_elem<Elem::f16>(a, head_dim, num_q_items, num_kv_items, stream);
  return launch_tile_bwd_elem<Elem::bf16>(a, head_dim, num_q_items, num_kv_items, stream);
}

}  // namespace esa
