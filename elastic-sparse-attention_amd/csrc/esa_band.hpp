// Device helpers shared by the band-gathered kernels (gfx950): slot
// layouts and swizzles, 16x16x32 MFMA, lane-group reductions, and each
// row's index list as per-entry ("band") keys with the group's band
// descriptors.
//
// MFMA 16x16x32 register layouts (gfx950):
//   A[i][k]: lane l holds i = l%16, k = 8*(l/16) + e, e = 0..7
//   B[k][j]: lane l holds k = 8*(l/16) + e, j = l%16
//   C[i][j]: lane l, reg r holds i = 4*(l/16) + r, j = l%16
// ds_read_b64_tr_b16 in each 16-lane group: lane g receives element r from
// lane 4r + g/4's 8-byte chunk, element g%4.
#pragma once
#include "esa_tile.hpp"

namespace esa {

typedef __attribute__((address_space(3))) uint16_t lds_u16;

template <int D>
struct BandCfg {
  static constexpr int NS = D / 32;       // QK^T k-steps (32 dims each)
  static constexpr int NV = D / 16;       // 16-dim slices of O^T
  static constexpr int CW = D / 4;        // dims per lane group of an O row
  static constexpr int CPR = D / 8;       // 16-byte chunks per K/V row
  static constexpr int ROWB = 2 * D;      // bytes per row
  static constexpr int SLOT = 16 * D;     // elements per V ring slot (16 rows)
  static constexpr int VLOADS = 16 * CPR / 64;  // DMA instructions per band
};

// physical 16-byte chunk of logical chunk lc in row r of a V slot: the 16
// lanes of a transposed read hit 16 distinct bank groups (at D = 256 a
// 16-lane group reads chunks 8 k + c, k = 0..3, of 4 rows: chunks 16 apart
// share a bank group, so bit 4 of the chunk also moves it; every form is its
// own inverse, as the DMA offsets need)
template <int D>
__device__ __forceinline__ int vswz(int r, int lc) {
  return D == 256 ? lc ^ (r & 3) ^ ((lc >> 4) << 2)
                  : (D == 128 ? lc ^ (r & 3) : lc ^ ((r >> 1) & 1));
}
// the same for a K slot: 16 lanes reading one chunk of rows 0..15 hit 16
// distinct bank groups
template <int D>
__device__ __forceinline__ int kswz(int r, int lc) {
  return D >= 128 ? lc ^ (r & 15) : lc ^ ((r >> 1) & 7);
}

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// max over the 4 lanes l, l^16, l^32, l^48 (one row's lanes), NaN if one of
// them is NaN (v_maximum3_f32: a row's NaN score, from a non-finite key it
// lists, must reach the row's softmax as the reference's does)
__device__ __forceinline__ float row4_max(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  const float m1 = __builtin_elementwise_maximum(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(m1), __float_as_uint(m1),
                                                  false, false);
  return __builtin_elementwise_maximum(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// row4_max of a and of b at once: the first swap pairs a's lanes l, l + 32
// in lanes 0..31 and b's in lanes 32..63, one l ^ 16 swap finishes both
// halves, and a last l ^ 32 swap hands each value to every lane (7 VALU
// instructions for the two instead of 12; the same maxima, NaN included)
__device__ __forceinline__ void row4_max2(float& a, float& b) {
  const auto s1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                   false);
  const float m1 = __builtin_elementwise_maximum(__uint_as_float(s1[0]), __uint_as_float(s1[1]));
  const auto s2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(m1), __float_as_uint(m1),
                                                   false, false);
  const float m2 = __builtin_elementwise_maximum(__uint_as_float(s2[0]), __uint_as_float(s2[1]));
  const auto s3 = __builtin_amdgcn_permlane32_swap(__float_as_uint(m2), __float_as_uint(m2),
                                                   false, false);
  a = __uint_as_float(s3[0]);
  b = __uint_as_float(s3[1]);
}

// min / max over the 16 lanes of a lane group (DPP row rotations)
// (a row rotation writes every lane, so the moves carry no old value and
// fold into the min / max as DPP operands)
__device__ __forceinline__ int row16_min(int v) {
  v = min(v, __builtin_amdgcn_mov_dpp(v, 0x128, 0xf, 0xf, true));
  v = min(v, __builtin_amdgcn_mov_dpp(v, 0x124, 0xf, 0xf, true));
  v = min(v, __builtin_amdgcn_mov_dpp(v, 0x122, 0xf, 0xf, true));
  v = min(v, __builtin_amdgcn_mov_dpp(v, 0x121, 0xf, 0xf, true));
  return v;
}
__device__ __forceinline__ int row16_max(int v) {
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0x128, 0xf, 0xf, true));
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0x124, 0xf, 0xf, true));
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0x122, 0xf, 0xf, true));
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0x121, 0xf, 0xf, true));
  return v;
}

// This lane's row i (of a 16-row group): slot (q, r), r = 0..15 of lane
// group q, holds entry j = (16 q + r + rot) mod 64, so a wave walking the
// slots in order visits the entries from entry rot on.  The row's key of
// that entry is -1 when the entry is masked (j >= w, idx > i) or the row is
// past q_len; the group's band descriptor of the slot is lo | W << 24, with
// lo / lo + W - 1 the smallest / largest valid key of the slot's entry over
// the group's rows (W = 0: no row uses it; W capped at 255); lo < 2^24 (host
// check).  Both come packed into 5 registers:
//   kd[r / 4], byte r % 4: the row's key of slot (q, r) minus the slot's lo,
//     0xFF for no key.  A band spans at most 31 keys over 16 rows (keys move
//     by at most 2 per row); an offset past 254 would read as no key, as a
//     tail pass bounded by the capped W would drop it.
//   info1: lane (n, q) holds the descriptor of slot (q, n), so slot (q, r)'s
//     is readlane(info1, 16 q + r).
// o_j is formed once per entry: entry j_r + 1 is j_{r+1} = (16 q + r + 1 +
// rot) mod 64 except at j_r = 63, whose o_64 is formed once.
//
// The rotation is the L2 schedule: groups are dispatched one after another
// onto an XCD's resident waves, each walking its 64 entries in the same
// time, so with rot = 0 the groups resident at once sit at every stage of
// their walk and touch the K/V rows of all 64 entries.  Starting each group
// at the entry the groups dispatched before it are at (rot growing by a
// little more than 64 / resident waves per dispatched group; the callers
// give their measured rates) keeps the resident groups on neighbouring
// entries, whose keys overlap: an L2 model of one XCD (4 MB LRU, 320
// resident waves) at B=1 H=32 L=32768 layer 4 puts the hit rate at 0.79
// without and 0.94 with the rotation.  That holds once waves are replaced
// one at a time; a grid of a few rounds starts each round at once, where
// the callers pass rot = 0 (band_rotation).
__device__ __forceinline__ void band_rows(const PatternConsts& pc, int h, int i, bool row_ok,
                                          int q, int n, int rot, uint32_t (&kd)[4],
                                          int& info1) {
  const HeadWeights hw = head_weights(pc, h);
  const RowParams rp = row_params(pc, i);
  int ov[17];
#pragma unroll
  for (int r = 0; r < 17; ++r) ov[r] = oversized(rp, (16 * q + r + rot) & 63);
  const int o64 = oversized(rp, 64);
  int kreg[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int j = (16 * q + r + rot) & 63;
    const int idx = interp_index(ov[r], j == 63 ? o64 : ov[r + 1], hw);
    kreg[r] = (row_ok && j < pc.w && idx <= i) ? idx : -1;
  }
  info1 = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) kd[w] = 0u;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int lo = row16_min(kreg[r] < 0 ? 0x7fffffff : kreg[r]);
    const int hi = row16_max(kreg[r]);
    const int wdt = hi >= 0 ? min(hi - lo + 1, 255) : 0;
    const int desc = hi >= 0 ? (lo | (wdt << 24)) : 0;
    info1 = n == r ? desc : info1;
    // kreg[r] - lo is in 0 .. 254 for a key in reach, and for no key
    // (kreg[r] = -1 <= lo - 1) wraps past 255 as unsigned
    const uint32_t db = min((uint32_t)(kreg[r] - lo), 0xFFu);
    kd[r >> 2] |= db << (8 * (r & 3));
  }
}

}  // namespace esa
