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
//   S^T = K Q^T    NS x v_mfma_f32_32x32x16_bf16 (A = K rows from LDS,
//                  B = Q kept in registers for the whole item)
//   softmax        online, in registers, log2 domain.  The S^T accumulator
//                  layout gives each lane one row and 16 of the block's keys;
//                  the mask enters as the accumulator's initial value (0 or
//                  -inf).  A block that holds no valid key for any row of the
//                  wave is skipped whole (K reads, both products, softmax).
//                  The running max is raised only when a row's
//                  block max exceeds it by more than 8 (log2), so the O
//                  rescale is rare; probabilities stay below 2^8.
//   O^T += V^T P^T 2 ND x v_mfma_f32_32x32x16_bf16 (A = V^T read with
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
template <int D, int BMQ>
__global__ __launch_bounds__(BMQ * 2, 2) void tile_fwd_kernel(TileArgs A) {
  using C = TileCfg<D, BMQ>;
  // stage buffers (HALF rows x D, rows unpadded, chunks swizzled); separate
  // objects, so the compiler can tell reads of one buffer from the direct
  // loads into the other
  __shared__ __attribute__((aligned(1024))) uint16_t k_st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t v_st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t k_st1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t v_st1[C::STAGE];
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

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hf = lane >> 5, l32 = lane & 31;

  const int i = qb * C::BM + wave * 32 + l32;  // this lane's query row = position
  const bool row_ok = i < A.q_len;

  // Q as the B operand of S^T = K Q^T: 8 consecutive d per lane and k-step.
  bf16x8 qop[C::NS];
  {
    const uint16_t* qrow = A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)i * A.qss;
#pragma unroll
    for (int s = 0; s < C::NS; ++s) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row_ok) raw = *(const u32x4*)(qrow + 16 * s + 8 * hf);
      qop[s] = __builtin_bit_cast(bf16x8, raw);
    }
  }

  // ---- this row's index list
  RowWalker walk;
  walk.init(A.pc, h, i, row_ok);

  float m_run = -INFINITY;  // running max, log2 units (the same in both halves)
  float l_run = 0.f;        // running sum of p over this lane's half of the keys (-> lse)
  float n_run = 0.f;        // the same sum of p rounded to bf16, as PV sees it (-> O)
  f32x16 oacc[C::ND];
#pragma unroll
  for (int d = 0; d < C::ND; ++d) oacc[d] = f32x16{};

  // ---- staging: buffer resources over this (batch, kv head)'s rows; keys at
  // or past kv_len are outside num_records and load as zeros (the host keeps
  // kv_len * row stride * 2 below 2^31)
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh), (short)0,
      (int)((int64_t)A.kv_len * A.kss * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh), (short)0,
      (int)((int64_t)A.kv_len * A.vss * 2), 0x00020000);
  // ---- LDS read addresses (elements), fixed for the whole item: K rows
  // 32 kbl + l32 at chunk 2 s + hf; V rows 4 hf + lam / 4 (+ 32 kbl + 16 u,
  // + 8) at column 32 d + 16 (g4 & 1) + 4 (lam & 3)
  const int g4 = lane >> 4, lam = lane & 15;
  int kaddr[C::NS], vaddr[C::ND];
#pragma unroll
  for (int s = 0; s < C::NS; ++s) kaddr[s] = l32 * D + 8 * ((2 * s + hf) ^ swz_k<D>(l32));
  {
    const int vrow = 4 * hf + (lam >> 2);
#pragma unroll
    for (int d = 0; d < C::ND; ++d) {
      const int col = 32 * d + 16 * (g4 & 1) + 4 * (lam & 3);
      vaddr[d] = vrow * D + 8 * ((col >> 3) ^ swz_v<D>(vrow)) + (col & 7);
    }
  }

  const float scale = A.scale_log2;  // > 0 (checked on the host)

  // One 32-key block: keys 32 kbl .. 32 kbl + 31 of a stage buffer (Kb, Vb),
  // whose valid-key bits for this row are mbits.
  auto block = [&](const uint16_t* Kb, const uint16_t* Vb, int kbl, uint32_t mbits) {
    // lane half hf holds keys 8*(r/4) + 4*hf + r%4 of the block
    const uint32_t mk = mbits >> (4 * hf);
    // a 32 x 32 block in which no row of the wave has a valid key contributes
    // p = 0 to every row: its reads, MFMAs and softmax are all skipped (O, the
    // running max and the sums are unchanged, bit for bit)
    if (!wave_any(mk != 0u)) return;

    // all K operand reads first, so their LDS latency overlaps
    bf16x8 ka[C::NS];
#pragma unroll
    for (int s = 0; s < C::NS; ++s) ka[s] = *(const bf16x8*)(Kb + kaddr[s] + 32 * kbl * D);
    // the mask enters as the accumulator's initial value: 0 for a valid key,
    // -inf for a masked one
    f32x16 sacc;
    mask_init<0>(sacc, ~mk);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < C::NS; ++s) sacc = mfma32(ka[s], qop[s], sacc);
    // the V^T operands of this block, read while the softmax runs
    s16x4 va[C::ND][4];
#pragma unroll
    for (int d = 0; d < C::ND; ++d) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint16_t* p1 = Vb + vaddr[d] + (32 * kbl + 16 * u) * D;
        va[d][2 * u] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p1);
        va[d][2 * u + 1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1 + 8 * D));
      }
    }
    __builtin_amdgcn_sched_barrier(0);

    uint32_t pw[8];  // P as packed bf16 pairs: pw[q] holds regs 2q, 2q+1
    // x = scaled score relative to the running max (log2 units); a masked
    // key stays -inf (scale > 0)
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float smax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = __builtin_fmaf(sacc[r], scale, -m_use);
      smax = fmaxf(smax, sacc[r]);
    }
    smax = half_max(smax);
    // raise the running max of a row when this block exceeds it by more
    // than the slack (or when the row sees its first valid key)
    const bool grow = m_run == -INFINITY ? smax != -INFINITY : smax > kRescaleSlack;
    if (wave_any(grow)) {
      const float delta = grow ? smax : 0.f;
      // rows that do not grow keep alpha = 1 (m_run may still be -inf there)
      const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - (m_use + delta)) : 1.0f;
      l_run *= alpha;
      n_run *= alpha;
#pragma unroll
      for (int d = 0; d < C::ND; ++d) oacc[d] *= alpha;
      m_run = grow ? m_use + delta : m_run;
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] -= delta;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float p0 = __builtin_amdgcn_exp2f(sacc[2 * q]);
      const float p1 = __builtin_amdgcn_exp2f(sacc[2 * q + 1]);
      l_run += p0;
      l_run += p1;
      pw[q] = pack_bf16x2(p0, p1);
      // normalise O by the probabilities PV actually used, so a row led by
      // one key reproduces that key's value row
      n_run = dot2_bf16(pw[q], n_run);
    }

#pragma unroll
    for (int d = 0; d < C::ND; ++d) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const s16x4 vv[2] = {va[d][2 * u], va[d][2 * u + 1]};
        const bf16x8 a = __builtin_bit_cast(bf16x8, vv);
        const u32x4 pq = {pw[4 * u], pw[4 * u + 1], pw[4 * u + 2], pw[4 * u + 3]};
        oacc[d] = mfma32(a, __builtin_bit_cast(bf16x8, pq), oacc[d]);
      }
    }
  };

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

  // ---- two stage buffers, one stage ahead: each barrier retires every
  // wave's reads of the other buffer before the next stage is loaded into it.
  // Stages go in pairs (buffer 0, buffer 1); this row's valid keys of both
  // are walked first.  The next two stage keys are read together at the top
  // of a pair (clamped indices: unconditional scalar loads, one wait).
  int ka = s0 < s1 ? stage_key0(s0) : 0;
  if (s0 < s1) issue(ka, k_st0, v_st0);
  for (int st = s0; st < s1; st += 2) {
    const bool has_b = st + 1 < s1, has_c = st + 2 < s1;
    const int kb = stage_key0(min(st + 1, s1 - 1));
    const int kc = stage_key0(min(st + 2, s1 - 1));
    uint32_t mb[2 * C::NB];
    walk.stage_pair<C::NB>(ka, kb, has_b, mb);

    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (has_b) issue(kb, k_st1, v_st1);
#pragma unroll
    for (int j = 0; j < C::NB; ++j) block(k_st0, v_st0, j, mb[j]);
    if (!has_b) break;

    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (has_c) issue(kc, k_st0, v_st0);
#pragma unroll
    for (int j = 0; j < C::NB; ++j) block(k_st1, v_st1, j, mb[C::NB + j]);
    ka = kc;
  }

  // ---- epilogue: normalise and store O rows and the log-sum-exp
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float n_tot = n_run + __shfl_xor(n_run, 32, 64);
  if (row_ok) {
    const float inv = n_tot > 0.f ? 1.f / n_tot : 0.f;
    uint16_t* orow = A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)i * A.oss;
#pragma unroll
    for (int d = 0; d < C::ND; ++d) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        bf16x4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = (__bf16)(oacc[d][4 * q4 + e] * inv);
        *(bf16x4*)(orow + 32 * d + 8 * q4 + 4 * hf) = ov;
      }
    }
    if (A.lse && hf == 0) {
      const float lse = l_tot > 0.f ? (m_run + __log2f(l_tot)) * 0.69314718055994530942f
                                    : -INFINITY;
      A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + i] = lse;
    }
  }
}

hipError_t launch_tile_fwd(const TileArgs& a, int head_dim, int64_t num_items,
                           hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  dim3 grid((unsigned)num_items);
  if (a.rows64) {
    if (head_dim == 128)
      tile_fwd_kernel<128, 64><<<grid, 128, 0, stream>>>(a);
    else
      tile_fwd_kernel<64, 64><<<grid, 128, 0, stream>>>(a);
  } else {
    if (head_dim == 128)
      tile_fwd_kernel<128, 128><<<grid, 256, 0, stream>>>(a);
    else
      tile_fwd_kernel<64, 128><<<grid, 256, 0, stream>>>(a);
  }
  return hipGetLastError();
}

}  // namespace esa
