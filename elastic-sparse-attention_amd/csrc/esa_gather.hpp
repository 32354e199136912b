// Per-row index sources shared by the gather forward, the naive-path weights
// and the gather backward: a query row's w entries either regenerated from
// the elastic pattern (bit-exact with elastic_sparse_attention.py:470-535,
// masked entries 0 and clamped to [0, kv_len - 1] as _triton_forward does,
// :602-615) or read from explicit index / mask arrays (the operator
// ElasticSparseAttentionFunction, :241-297).
#pragma once
#include "esa_elem.hpp"
#include "esa_internal.hpp"

namespace esa {

struct RowEntries {
  HeadWeights hw;
  RowParams rp;
  int pos;       // the row's query position
  bool bad_pos;  // a position outside [-kv_len, kv_len): the row reads NaN

  template <bool PATTERN>
  __device__ __forceinline__ void init(const IndexSource& S, int h, int r) {
    pos = r;
    bad_pos = false;
    hw = HeadWeights{};
    rp = RowParams{};
    if (PATTERN) {
      if (S.positions) {
        // negative positions count from the end, as torch indexing does
        const int64_t p0 = S.positions[r];
        const int64_t p64 = p0 < 0 ? p0 + S.kv_len : p0;
        bad_pos = p64 < 0 || p64 >= S.kv_len;
        pos = bad_pos ? 0 : (int)p64;
      }
      hw = head_weights(S.pc, h);
      rp = row_params(S.pc, pos);
    }
  }

  // Entry j < w of the row: its key and whether it is valid.  A pattern key
  // is always in [0, kv_len); an explicit one may lie outside (the Triton
  // kernel then scores it 0 against zero K/V, :131-134).
  template <bool PATTERN>
  __device__ __forceinline__ void entry(const IndexSource& S, int h, int r, int j, bool& valid,
                                        int64_t& key) const {
    if (PATTERN) {
      const int idx = interp_index(oversized(rp, j), oversized(rp, j + 1), hw);
      valid = idx <= pos;
      int kk = valid ? idx : 0;
      kk = kk < 0 ? 0 : (kk > S.kv_len - 1 ? S.kv_len - 1 : kk);
      key = kk;
    } else {
      key = load_int_any(S.indices, S.index_bytes, (int64_t)h * S.ish + (int64_t)r * S.iss + j);
      valid = load_int_any(S.mask, S.mask_bytes, (int64_t)h * S.msh + (int64_t)r * S.mss + j) != 0;
    }
  }
};

// Dropout multiplier of entry j of row (b, h, r): 1 without dropout, else 0
// or 1 / (1 - p_drop) by the counter-based keep decision.
__device__ __forceinline__ float drop_factor(const DropoutArgs& dr, int b, int h, int r, int j,
                                             int H, int q_len, int w) {
  if (!(dr.p > 0.f)) return 1.f;
  const uint64_t idx = (((uint64_t)b * H + h) * (uint64_t)q_len + r) * (uint64_t)w + j;
  return dropout_keep(dr.seed, idx, dr.p) ? dr.scale : 0.f;
}

// Sum over aligned groups of N lanes (N = 8, 16, 32, 64), in every lane of
// the group: DPP within 16-lane rows (quad swaps and a half-row mirror for
// N = 8, row rotations by 8, 4, 2, 1 for 16), cross-row steps by shuffles.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  auto dpp = [](float x, int ctrl) -> float {
    switch (ctrl) {  // the control word must be a constant
      case 0xB1: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));
      case 0x4E: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));
      case 0x141: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false));
      case 0x128: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
      case 0x124: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xf, 0xf, false));
      case 0x122: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x122, 0xf, 0xf, false));
      default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xf, 0xf, false));
    }
  };
  if (N == 8) {
    v += dpp(v, 0xB1);   // quad_perm [1, 0, 3, 2]
    v += dpp(v, 0x4E);   // quad_perm [2, 3, 0, 1]
    v += dpp(v, 0x141);  // row_half_mirror: the other quad of the 8
    return v;
  }
  v += dpp(v, 0x128);  // row_ror 8
  v += dpp(v, 0x124);  // row_ror 4
  v += dpp(v, 0x122);  // row_ror 2
  v += dpp(v, 0x121);  // row_ror 1
  if (N >= 32) v += __shfl_xor(v, 16, 64);
  if (N >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// Orders LDS writes of a wave before its later reads (the wave's lanes run
// in lock step; the fences keep the compiler from reordering).
__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace esa
