// Block-sparse flash-attention forward over the elastic pattern (gfx950).
//
// Replaces the forward branch of the reference's per-token Triton kernel
// (elastic_sparse_attention.py:117-166) for prefill.  One workgroup (4 waves,
// 256 lanes) owns one (batch, head, 128-row query block) work item and visits
// only the key blocks the block layout lists as active for it.  Inside a
// staged block each wave issues MFMAs only for the 32 x 32 (rows x keys)
// blocks where one of its rows has a valid key (about 36% of those in active
// 128 x 128 tiles at dilated layers), since the others contribute exactly
// zero.
//
// K/V staging: keys are consumed in 64-key stages.  With a layout built at
// 64-key blocks (the 128-key tiles split in halves, a half listed only when a
// row of the query block has a valid key in it) each listed block is one
// stage; a 128-key layout gives two stages per tile.  Each stage's K and V
// rows are copied HBM -> LDS by buffer_load_dwordx4 ... lds (no registers),
// one stage ahead, into two stage buffers (64 KB per workgroup at D = 128, so
// two workgroups share a CU).  Rows past kv_len fall outside the buffer
// resource and read as zeros.  Within a buffer, 16-byte chunks of a row are
// XOR-swizzled (K: 16 consecutive rows hit 16 distinct bank groups for the
// 16-byte MFMA operand reads; V: the 4 rows of a ds_read_b64_tr_b16 group hit
// distinct bank groups), since the direct loads write whole rows unpadded.
//
// Per stage and wave (32 query rows):
//   mask           each lane owns one query row; rows whose index list is a
//                  contiguous run (the sliding window of layer 0, and the
//                  first w - 1 rows of every layer) set a bit range, the
//                  others walk their elastic indices (the same float32
//                  sequence as the layout builder) through the stage
// then for each 32-key block of the stage:
//   S^T = K Q^T    NS x v_mfma_f32_32x32x16_{bf16,f16} (A = K rows from LDS,
//                  B = Q kept in registers for the whole item)
//   softmax        online, in registers, log2 domain.  The S^T accumulator
//                  layout gives each lane one row and 16 of the block's keys;
//                  the mask enters as the accumulator's initial value (0 or
//                  -inf).  A block that holds no valid key for any row of the
//                  wave is skipped whole (K reads, both products, softmax).
//                  The running max is raised only when a row's
//                  block max exceeds it by more than 8 (log2), so the O
//                  rescale is rare; probabilities stay below 2^8.
//   O^T += V^T P^T 2 ND x v_mfma_f32_32x32x16_{bf16,f16} (A = V^T read with
//                  ds_read_b64_tr_b16 from row-major V in LDS, B = P straight
//                  from the S^T accumulators: a key permutation shared by
//                  both operands leaves the contraction unchanged)
//
// MFMA 32x32x16 register layouts (gfx950):
//   A[i][k]: lane l holds i = l%32, k = 8*(l/32) + e, e = 0..7
//   B[k][j]: lane l holds k = 8*(l/32) + e, j = l%32
//   C[i][j]: lane l, reg r holds i = 8*(r/4) + 4*(l/32) + r%4, j = l%32
// ds_read_b64_tr_b16 in each 16-lane group: lane g receives element r from
// lane 4r + g/4's 8-byte chunk, element g%4.
// buffer_load_dwordx4 ... lds: lane l's 16 bytes land at M0 + 16 l; offsets
// (voffset + soffset) at or past num_records read as zero.
#include "esa_tile.hpp"

namespace esa {

// BMQ query rows per work item: 128 (4 waves, 64-key stages, two
// workgroups per CU) or 64 (2 waves, 32-key stages, four workgroups per CU:
// fewer waves meet at each barrier)
template <int D, int BMQ>
struct TileCfg {
  static constexpr int BM = BMQ;
  static constexpr int W = BMQ / 32;              // waves
  static constexpr int HALF = BMQ == 128 ? 64 : 32;  // keys per stage
  static constexpr int LOG_HALF = BMQ == 128 ? 6 : 5;
  static constexpr int NB = HALF / 32;            // 32-key blocks per stage
  static constexpr int CPR = D / 8;               // 16-byte chunks per row
  static constexpr int STAGE = HALF * D;          // elements per stage buffer (one matrix)
  static constexpr int LOADS = HALF * CPR / (64 * W);  // 16-byte loads per lane per matrix per stage
  static constexpr int NS = D / 16;               // k-steps of QK^T
  static constexpr int ND = D / 32;               // 32-wide d blocks of PV
  static_assert(LOADS >= 1 && LOADS * 64 * W == HALF * CPR, "whole stage per load round");
};

// (the second launch bound is the minimum number of waves per SIMD: two,
// so at most 256 VGPRs; LDS then allows two 128-row or four 64-row
// workgroups per CU)
//
// PRE: each row's valid keys per stage come from A.smask (written once per
// layout by stage_mask_kernel: the same bits the walk below computes, for a
// layout whose stages are its key blocks), one load per stage instead of
// the index walk, which at dilated layers costs about a third of the
// kernel's VALU work and is the same for every batch element.
template <int D, int BMQ, Elem E, bool PRE>
__global__ __launch_bounds__(BMQ * 2, D == 64 ? 4 : 2) void tile_fwd_kernel(TileArgs A) {
  using C = TileCfg<D, BMQ>;
  // stage buffers (HALF rows x D, rows unpadded, chunks swizzled); separate
  // objects, so the compiler can tell reads of one buffer from the direct
  // loads into the other
  __shared__ __attribute__((aligned(1024))) uint16_t k_st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t v_st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t k_st1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t v_st1[C::STAGE];
  __shared__ uint32_t wave_met[C::W];  // each wave's non-finite flag (below)
  // the layout and the work list are read-only here: scalar loads
  const cptr_i32 items = (cptr_i32)A.items;
  const cptr_i32 row_ptr = (cptr_i32)A.row_ptr;
  const cptr_i32 col_idx = (cptr_i32)A.col_idx;

  // ---- work item (uniform over the workgroup; -1 pads the XCD runs)
  const int item = items[blockIdx.x];
  if (item < 0 || item >= A.num_bh * A.nqb) return;
  const int qb = item % A.nqb;
  if (qb >= A.nq) return;
  const int bh = item / A.nqb;
  const int h = bh % A.H;
  const int b = bh / A.H;
  const int kvh = h / A.groups;

  // ---- the item: set-up, the stages, the store.  An item whose outputs met
  // a non-finite value (an Inf or NaN in V, staged with a 32-key block, can
  // reach rows that do not list it through 0 * Inf in PV) runs again, every
  // wave of the workgroup together, with the V operands sanitised (SAN):
  // rows whose entries bring no non-finite value then get exactly the bits a
  // run without it gives, and the reference's non-finite values go back in
  // after the store.  Each run sets itself up from the kernel arguments, so
  // nothing but the flag is live from one to the other, and the second costs
  // the first no registers.
  auto run_item = [&](auto san_tag) -> bool {
    constexpr bool SAN = decltype(san_tag)::value;
    // (the lane id passes through an empty asm, so the compiler cannot share
    // the runs' per-lane set-up and keep it live from one to the other)
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;

    const int i = qb * C::BM + wave * 32 + l32;  // this lane's query row = position
    const bool row_ok = i < A.q_len;

    Rows32<D, E> rows;
    rows.init(lane, A.scale_log2);  // scale > 0 (checked on the host)
    rows.load_q(A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)i * A.qss, row_ok);

    // ---- this row's index list
    RowWalker walk;
    if constexpr (!PRE) walk.init(A.pc, h, i, row_ok);

    // ---- staging: buffer resources over this (batch, kv head)'s rows; keys at
    // or past kv_len are outside num_records and load as zeros (the host keeps
    // kv_len * row stride * 2 below 2^31)
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh), (short)0,
        (int)((int64_t)A.kv_len * A.kss * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh), (short)0,
        (int)((int64_t)A.kv_len * A.vss * 2), 0x00020000);

    const int64_t lrow = (int64_t)h * A.nqb + qb;
    // ---- the item's 64-key stages: layout key blocks of 64 keys are one stage
    // each; 128-key blocks are two (stage s is half s & 1 of block s >> 1)
    const int sh = A.stage_shift;
    const int s0 = row_ptr[lrow] << sh, s1 = row_ptr[lrow + 1] << sh;

    // load j of this lane fills chunk slot (LOADS wave + j) * 64 + lane of a
    // stage buffer: row slot / CPR, physical chunk slot % CPR
    int koff[C::LOADS], voff[C::LOADS];
  #pragma unroll
    for (int j = 0; j < C::LOADS; ++j) {
      const int slot = (C::LOADS * wave + j) * 64 + lane;
      const int row = slot / C::CPR, pc = slot % C::CPR;
      koff[j] = (row * (int)A.kss + 8 * (pc ^ swz_k<D>(row))) * 2;
      voff[j] = (row * (int)A.vss + 8 * (pc ^ swz_v<D>(row))) * 2;
    }
    auto stage_key0 = [&](int st) {
      return (col_idx[st >> sh] << (C::LOG_HALF + sh)) + ((st & sh) << C::LOG_HALF);
    };
    // the HALF keys from key0 -> buffers (kd, vd)
    auto issue = [&](int key0, uint16_t* kd, uint16_t* vd) {
      const int ks = key0 * (int)A.kss * 2, vs = key0 * (int)A.vss * 2;
  #pragma unroll
      for (int j = 0; j < C::LOADS; ++j) {
        // each load writes 64 lanes x 16 bytes = 512 elements
        load_lds16(krs, kd + (C::LOADS * wave + j) * 512, koff[j], ks);
        load_lds16(vrs, vd + (C::LOADS * wave + j) * 512, voff[j], vs);
      }
    };

    // the rerun: this lane's 16-byte chunks of a landed V stage (the ones its
  // DMAs wrote) with non-finite values replaced by +0, before the barrier
  // that hands the stage to the blocks
  auto sanitize_stage = [&](uint16_t* vd) {
#pragma unroll
    for (int j = 0; j < C::LOADS; ++j) {
      u32x4* p = (u32x4*)(vd + (C::LOADS * wave + j) * 512) + lane;
      u32x4 x = *p;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = sanitize2<E>(x[e]);
      *p = x;
    }
  };

  // PRE: this row's mask words of stages st (and st + 1 if has_b) -> mb;
    // zeros for rows past q_len, as the walk gives them
    const int64_t mrow = (int64_t)(wave * 32 + l32) * C::NB;
    auto load_masks = [&](int st, bool has_b, uint32_t (&mb)[2 * C::NB]) {
      const uint32_t* m0 = A.smask + (int64_t)st * (C::BM * C::NB) + mrow;
  #pragma unroll
      for (int j = 0; j < C::NB; ++j) {
        mb[j] = row_ok ? m0[j] : 0u;
        mb[C::NB + j] = row_ok && has_b ? m0[C::BM * C::NB + j] : 0u;
      }
    };
    // ---- the item's stages
    uint32_t mnext[2 * C::NB];
    if constexpr (PRE) {
      if (s0 < s1) load_masks(s0, s0 + 1 < s1, mnext);
    }
    // ---- two stage buffers, one stage ahead: each barrier retires every
    // wave's reads of the other buffer before the next stage is loaded into it.
    // Stages go in pairs (buffer 0, buffer 1); this row's valid keys of both
    // are walked first (or, with PRE, were loaded during the previous pair).
    // The next two stage keys are read together at the top of a pair (clamped
    // indices: unconditional scalar loads, one wait).
    int ka = s0 < s1 ? stage_key0(s0) : 0;
    if (s0 < s1) issue(ka, k_st0, v_st0);
    for (int st = s0; st < s1; st += 2) {
      const bool has_b = st + 1 < s1, has_c = st + 2 < s1;
      const int kb = stage_key0(min(st + 1, s1 - 1));
      const int kc = stage_key0(min(st + 2, s1 - 1));
      uint32_t mb[2 * C::NB];
      if constexpr (PRE) {
  #pragma unroll
        for (int j = 0; j < 2 * C::NB; ++j) mb[j] = mnext[j];
      } else {
        walk.stage_pair<C::NB>(ka, kb, has_b, mb);
      }

      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      if constexpr (SAN) {
        sanitize_stage(v_st0);  // (this wave's own DMAs have landed)
        __builtin_amdgcn_s_waitcnt(0);
      }
      __syncthreads();
      if (has_b) issue(kb, k_st1, v_st1);
      // the next pair's masks, in flight during this pair's blocks (the waits
      // above the next barriers cover them)
      if constexpr (PRE) {
        if (has_c) load_masks(st + 2, st + 3 < s1, mnext);
      }
  #pragma unroll
      for (int j = 0; j < C::NB; ++j) rows.template block<SAN>(k_st0, v_st0, j, mb[j]);
      if (!has_b) break;

      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      if constexpr (SAN) {
        sanitize_stage(v_st1);
        __builtin_amdgcn_s_waitcnt(0);
      }
      __syncthreads();
      if (has_c) issue(kc, k_st0, v_st0);
  #pragma unroll
      for (int j = 0; j < C::NB; ++j) rows.template block<SAN>(k_st1, v_st1, j, mb[C::NB + j]);
      ka = kc;
    }

    // ---- epilogue: normalise and store O rows and the log-sum-exp
    const bool met_nonfinite = !SAN && !sum_finite(rows.oacc);
    uint16_t* const orow = A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)i * A.oss;
    rows.store(orow, A.lse ? A.lse + (int64_t)b * A.lsb + (int64_t)h * A.lsh + i : nullptr,
               row_ok);
    if (SAN && row_ok)
      rows.put_nonfinite(orow, A.pc, h, i, A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh, A.vss);
    return met_nonfinite;
  };
  const bool met = run_item(std::integral_constant<bool, false>{});
  // every wave's flag through its own LDS word and one barrier (which also
  // retires every wave's reads of the stage buffers before a rerun refills
  // them)
  const uint32_t wmet = wave_any(met) ? 1u : 0u;
  if ((threadIdx.x & 63) == 0) wave_met[threadIdx.x >> 6] = wmet;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint32_t any = 0u;
#pragma unroll
  for (int w = 0; w < C::W; ++w) any |= wave_met[w];
  if (any) run_item(std::integral_constant<bool, true>{});
}

template <Elem E, bool PRE>
void launch_tile_pre(const TileArgs& a, int head_dim, dim3 grid, hipStream_t stream) {
  if (a.rows64) {
    if (head_dim == 128)
      tile_fwd_kernel<128, 64, E, PRE><<<grid, 128, 0, stream>>>(a);
    else
      tile_fwd_kernel<64, 64, E, PRE><<<grid, 128, 0, stream>>>(a);
  } else {
    if (head_dim == 128)
      tile_fwd_kernel<128, 128, E, PRE><<<grid, 256, 0, stream>>>(a);
    else
      tile_fwd_kernel<64, 128, E, PRE><<<grid, 256, 0, stream>>>(a);
  }
}

template <Elem E>
void launch_tile_elem(const TileArgs& a, int head_dim, dim3 grid, hipStream_t stream) {
  if (a.smask)
    launch_tile_pre<E, true>(a, head_dim, grid, stream);
  else
    launch_tile_pre<E, false>(a, head_dim, grid, stream);
}

// One workgroup per (head, query block) of a 64 x 32, 128 x 64 or 128 x 128
// layout, one lane per query row: each lane walks its row's index list
// through the block's stages (the key blocks col_idx lists, ascending) as
// the forward does and stores the valid-key bits, word q of stage st for row
// r at masks[(st * BMQ + r) * NW + q].  Rows past the pattern get zeros.
template <int BMQ, int NW>
__global__ __launch_bounds__(BMQ) void stage_mask_kernel(PatternConsts pc, int nqb, int seq_len,
                                                         int log_bn, const int32_t* row_ptr,
                                                         const int32_t* col_idx,
                                                         uint32_t* masks) {
  const int item = blockIdx.x;  // h * nqb + qb
  const int h = item / nqb, qb = item % nqb;
  const int r = threadIdx.x, i = qb * BMQ + r;
  RowWalker walk;
  walk.init(pc, h, i, i < seq_len);
  const int s0 = row_ptr[item], s1 = row_ptr[item + 1];
  for (int st = s0; st < s1; ++st) {
    uint32_t mb[NW];
    walk.span<NW>(col_idx[st] << log_bn, mb);
#pragma unroll
    for (int q = 0; q < NW; ++q) masks[((int64_t)st * BMQ + r) * NW + q] = mb[q];
  }
}

hipError_t launch_stage_masks(const PatternConsts& pc, const LayoutDims& ld, const int32_t* row_ptr,
                              const int32_t* col_idx, uint32_t* masks, hipStream_t stream) {
  const int64_t items = (int64_t)pc.H * ld.nqb;
  if (items <= 0) return hipSuccess;
  dim3 grid((unsigned)items);
  if (ld.bm == 64)
    stage_mask_kernel<64, 1><<<grid, 64, 0, stream>>>(pc, ld.nqb, ld.seq_len, 5, row_ptr, col_idx,
                                                       masks);
  else if (ld.bn == 64)
    stage_mask_kernel<128, 2><<<grid, 128, 0, stream>>>(pc, ld.nqb, ld.seq_len, 6, row_ptr,
                                                         col_idx, masks);
  else  // 128 x 128 tiles (the backward's dQ)
    stage_mask_kernel<128, 4><<<grid, 128, 0, stream>>>(pc, ld.nqb, ld.seq_len, 7, row_ptr,
                                                         col_idx, masks);
  return hipGetLastError();
}

hipError_t launch_tile_fwd(const TileArgs& a, int head_dim, int64_t num_items,
                           hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  dim3 grid((unsigned)num_items);
  if (a.elem == (int)Elem::f16)
    launch_tile_elem<Elem::f16>(a, head_dim, grid, stream);
  else
    launch_tile_elem<Elem::bf16>(a, head_dim, grid, stream);
  return hipGetLastError();
}

}  // namespace esa
