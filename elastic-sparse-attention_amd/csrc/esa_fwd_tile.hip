// Block-sparse flash-attention forward over the elastic pattern (gfx950).
//
// Replaces the forward branch of the reference's per-token Triton kernel
// (elastic_sparse_attention.py:117-166) for prefill.  One workgroup (4 waves,
// 256 lanes) owns one (batch, head, 128-row query block) work item and visits
// only the 128-key tiles the block layout lists as active for it.
//
// Per tile and wave (32 query rows):
//   S^T = K Q^T    32 x v_mfma_f32_32x32x16_bf16 (A = K rows from LDS,
//                  B = Q kept in registers for the whole item)
//   mask           each lane regenerates its row's elastic indices inside the
//                  tile (the same float32 sequence as the layout builder)
//   softmax        online, per lane: the S^T accumulator layout gives every
//                  lane one query row (lane % 32) and 64 of the tile's keys,
//                  so the row max needs one cross-half exchange and nothing
//                  else; the running max and sum stay in registers
//   O^T += V^T P^T 32 x v_mfma_f32_32x32x16_bf16 (A = V^T read with
//                  ds_read_b64_tr_b16 from row-major V in LDS, B = P straight
//                  from the S^T accumulators: a key permutation shared by
//                  both operands leaves the contraction unchanged)
//
// MFMA 32x32x16 register layouts (checked on gfx950):
//   A[i][k]: lane l holds i = l%32, k = 8*(l/32) + e, e = 0..7
//   B[k][j]: lane l holds k = 8*(l/32) + e, j = l%32
//   C[i][j]: lane l, reg r holds i = 8*(r/4) + 4*(l/32) + r%4, j = l%32
// ds_read_b64_tr_b16 in each 16-lane group: lane g receives element r from
// lane 4r + g/4's 8-byte chunk, element g%4.
#include "esa_internal.hpp"

namespace esa {

template <int D>
struct TileCfg {
  static constexpr int BM = 128;
  static constexpr int BN = 128;
  static constexpr int KSTR = D + 8;   // K row pitch (elements): conflict-free b128 reads
  static constexpr int VSTR = D + 16;  // V row pitch: conflict-free transposed reads
  static constexpr int NS = D / 16;    // k-steps of QK^T
  static constexpr int ND = D / 32;    // 32-wide d blocks of PV
  static constexpr int CPR = D / 8;    // 16-byte chunks per row
  static constexpr int RPP = 256 / CPR;  // rows staged per pass
};

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <int D>
__global__ __launch_bounds__(256, 2) void tile_fwd_kernel(TileArgs A) {
  using C = TileCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[C::BN * C::KSTR];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[C::BN * C::VSTR];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int hf = lane >> 5, l32 = lane & 31;

  const int item = A.items[blockIdx.x];
  const int qb = item % A.nqb;
  const int bh = item / A.nqb;
  const int h = bh % A.H;
  const int b = bh / A.H;
  const int kvh = h / A.groups;

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

  const HeadWeights hw = head_weights(A.pc, h);
  const RowParams rp = row_params(A.pc, i);
  int jp = row_ok ? 0 : A.pc.w;  // next unread entry of this row's index list
  int o_cur = rp.st;             // o_jp

  float m_run = -INFINITY;  // running max, log2 units
  float l_run = 0.f;        // running sum over this lane's half of the keys
  f32x16 oacc[C::ND];
#pragma unroll
  for (int d = 0; d < C::ND; ++d) oacc[d] = f32x16{};

  const uint16_t* kg = A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh;
  const uint16_t* vg = A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh;
  const int64_t lrow = (int64_t)h * A.nqb + qb;
  const int t0 = A.row_ptr[lrow], t1 = A.row_ptr[lrow + 1];

  for (int t = t0; t < t1; ++t) {
    const int k0 = A.col_idx[t] * C::BN;

    // ---- stage the K and V tiles (row-major) in LDS; rows past kv_len are 0
#pragma unroll
    for (int p = 0; p < C::BN / C::RPP; ++p) {
      const int r = p * C::RPP + tid / C::CPR, c = tid % C::CPR;
      const int key = k0 + r;
      u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
      if (key < A.kv_len) {
        kv = *(const u32x4*)(kg + (int64_t)key * A.kss + 8 * c);
        vv = *(const u32x4*)(vg + (int64_t)key * A.vss + 8 * c);
      }
      *(u32x4*)(Ks + r * C::KSTR + 8 * c) = kv;
      *(u32x4*)(Vs + r * C::VSTR + 8 * c) = vv;
    }
    __syncthreads();

    // ---- S^T = K Q^T: block kb holds keys 32kb..32kb+31 x this wave's 32 rows
    f32x16 sacc[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      sacc[kb] = f32x16{};
#pragma unroll
      for (int s = 0; s < C::NS; ++s) {
        const bf16x8 a = *(const bf16x8*)(Ks + (32 * kb + l32) * C::KSTR + 16 * s + 8 * hf);
        sacc[kb] = mfma32(a, qop[s], sacc[kb]);
      }
    }

    // ---- this row's valid keys inside [k0, k0 + 128) as a 128-bit mask
    uint32_t mb0 = 0u, mb1 = 0u, mb2 = 0u, mb3 = 0u;
    while (jp < A.pc.w) {
      const int o_next = oversized(rp, jp + 1);
      const int idx = interp_index(o_cur, o_next, hw);
      if (idx > i) {  // indices rise with j: every later entry is masked too
        jp = A.pc.w;
        break;
      }
      if (idx >= k0 + C::BN) break;
      const int rel = idx - k0;
      if (rel >= 0) {
        const uint32_t bit = 1u << (rel & 31);
        const int wsel = rel >> 5;
        mb0 |= wsel == 0 ? bit : 0u;
        mb1 |= wsel == 1 ? bit : 0u;
        mb2 |= wsel == 2 ? bit : 0u;
        mb3 |= wsel == 3 ? bit : 0u;
      }
      o_cur = o_next;
      ++jp;
    }
    // lane half hf holds keys 32kb + 8*(r/4) + 4*hf + r%4: pre-shift by 4*hf
    const uint32_t mk[4] = {mb0 >> (4 * hf), mb1 >> (4 * hf), mb2 >> (4 * hf), mb3 >> (4 * hf)};

    // ---- online softmax (log2 domain)
    float smax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool on = (mk[kb] >> (8 * (r / 4) + (r % 4))) & 1u;
        const float s = on ? sacc[kb][r] * A.scale_log2 : -INFINITY;
        sacc[kb][r] = s;
        smax = fmaxf(smax, s);
      }
    }
    smax = fmaxf(smax, __shfl_xor(smax, 32, 64));
    const float m_new = fmaxf(m_run, smax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float psum = 0.f;
    bf16x8 pb[4][2];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(sacc[kb][r] - m_use);
        psum += p;
        pb[kb][r / 8][r % 8] = (__bf16)p;
      }
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int d = 0; d < C::ND; ++d) oacc[d] *= alpha;

    // ---- O^T += V^T P^T
    const int g = lane >> 4, lam = lane & 15;
#pragma unroll
    for (int d = 0; d < C::ND; ++d) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int key = 32 * kb + 16 * u + 4 * hf + (lam >> 2);
          const int col = 32 * d + 16 * (g & 1) + 4 * (lam & 3);
          const uint16_t* p1 = Vs + key * C::VSTR + col;
          const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p1);
          const s16x4 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1 + 8 * C::VSTR));
          const s16x4 vv[2] = {v1, v2};
          const bf16x8 a = __builtin_bit_cast(bf16x8, vv);
          oacc[d] = mfma32(a, pb[kb][u], oacc[d]);
        }
      }
    }
    __syncthreads();
  }

  // ---- epilogue: normalise and store O rows and the log-sum-exp
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (row_ok) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    uint16_t* orow = A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)i * A.oss;
#pragma unroll
    for (int d = 0; d < C::ND; ++d) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        bf16x4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = (__bf16)(oacc[d][4 * g4 + e] * inv);
        *(bf16x4*)(orow + 32 * d + 8 * g4 + 4 * hf) = ov;
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
  if (head_dim == 128)
    tile_fwd_kernel<128><<<grid, 256, 0, stream>>>(a);
  else
    tile_fwd_kernel<64><<<grid, 256, 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace esa
