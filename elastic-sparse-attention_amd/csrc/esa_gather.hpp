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

// One query row (b, h, r) of the per-row gather forward, by one wave (the
// body of gather_rows_kernel, esa_fwd_gather.hip, which describes it; also
// the band forward's path for rows whose positions are not consecutive):
// D = 64, 128 or 256 with 16-byte aligned rows; sc: 64 floats of LDS private
// to the wave.
template <Elem E, int D, bool PATTERN>
__device__ __forceinline__ void gather_one_row(const GatherArgs& A, int b, int h, int r,
                                               float* sc, int lane) {
  using T = typename ElemT<E>::T;
  constexpr int EPL = ElemT<E>::kPerChunk;  // elements per lane per load
  constexpr int LPK = D / EPL;              // lanes per row
  constexpr int KPI = 64 / LPK;             // rows per load instruction
  constexpr int SK = 16 * KPI < 64 ? 16 * KPI : 64;  // keys per chunk
  constexpr int NI = SK / KPI;              // load instructions per chunk
  static_assert(LPK <= 64 && 64 % LPK == 0 && NI <= 16, "row split");
  const int kvh = h / A.groups;
  const int gk = lane / LPK;  // row of an instruction this lane loads
  const int ln = lane % LPK;  // its 16-byte piece: elements EPL ln .. + EPL

  float qv[EPL];
  {
    const T* qrow = (const T*)A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)r * A.qss;
    const u32x4 raw = *(const u32x4*)(qrow + EPL * ln);
#pragma unroll
    for (int e = 0; e < EPL; ++e) qv[e] = ElemT<E>::chunk(raw, e);
  }
  const T* kbase = (const T*)A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh + EPL * ln;
  const T* vbase = (const T*)A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh + EPL * ln;
  RowEntries row;
  row.init<PATTERN>(A.src, h, r);

  auto dot16 = [&](const u32x4& raw) {
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc += qv[e] * ElemT<E>::chunk(raw, e);
    return acc;
  };

  float m = -INFINITY, l = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  const int w = A.src.w;
  for (int c0 = 0; c0 < w; c0 += SK) {
    // slot `lane` of the chunk: entry c0 + lane
    const int j = c0 + lane;
    bool valid = false;
    int64_t key = 0;
    if (lane < SK && j < w) row.entry<PATTERN>(A.src, h, r, j, valid, key);
    const bool in_range = key >= 0 && key < A.kv_len;
    const int kaddr = (valid && in_range) ? (int)key : 0;  // a row that exists
    u32x4 kd[NI], vd[NI];
#pragma unroll
    for (int t = 0; t < NI; ++t) {
      const int kk = __shfl(kaddr, KPI * t + gk, 64);
      kd[t] = *(const u32x4*)(kbase + (int64_t)kk * A.kss);
      vd[t] = *(const u32x4*)(vbase + (int64_t)kk * A.vss);
    }
#pragma unroll
    for (int t = 0; t < NI; ++t) {
      const float part = group_sum<LPK>(dot16(kd[t]));
      if (ln == 0) sc[KPI * t + gk] = part;
    }
    wave_sync_lds();
    float s = -INFINITY;
    if (lane < SK && valid) s = in_range ? sc[lane] * A.sm_scale : 0.f;
    const float cmax = wave_max(s);
    const float m_new = fmaxf(m, cmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float p = valid ? expf(s - m_use) : 0.f;
    const float alpha = expf(m - m_use);
    l = l * alpha + wave_sum(p);
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] *= alpha;
    m = m_new;
    wave_sync_lds();
    // PV weight of the slot (dropout keep factor applied)
    if (lane < SK) {
      const float keep = j < w ? drop_factor(A.drop, b, h, r, j, A.H, A.q_len, w) : 0.f;
      sc[lane] = (valid && in_range) ? p * keep : 0.f;
    }
    wave_sync_lds();
#pragma unroll
    for (int t = 0; t < NI; ++t) {
      const float pt = sc[KPI * t + gk];
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] += pt * ElemT<E>::chunk(vd[t], e);
    }
    wave_sync_lds();
  }
  // the KPI row groups' partial sums: lanes ln, ln + LPK, ...
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1)
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] += __shfl_xor(acc[e], off, 64);

  const float inv = row.bad_pos ? __builtin_nanf("") : (l > 0.f ? 1.f / l : 0.f);
  if (gk == 0) {
    T* orow = (T*)A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)r * A.oss + EPL * ln;
    float x[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) x[e] = acc[e] * inv;
    *(u32x4*)orow = ElemT<E>::pack_chunk(x);
  }
  if (A.lse && lane == 0)
    A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + r] =
        row.bad_pos ? __builtin_nanf("") : (l > 0.f ? m + logf(l) : -INFINITY);
}

// dot(q, k_row) over D (D % 4 == 0); q in LDS as float
template <Elem E>
__device__ __forceinline__ float row_dot(const float* __restrict__ qs,
                                         const typename ElemT<E>::T* __restrict__ kr, int D) {
  float acc = 0.f;
  if constexpr (E == Elem::f32) {
    for (int d = 0; d < D; d += 4) {
      const f32x4 kv = *(const f32x4*)(kr + d);
      acc += qs[d] * kv[0];
      acc += qs[d + 1] * kv[1];
      acc += qs[d + 2] * kv[2];
      acc += qs[d + 3] * kv[3];
    }
  } else {
    for (int d = 0; d < D; d += 4) {
      const u32x2 kv = *(const u32x2*)(kr + d);
      const u32x4 raw = {kv[0], kv[1], 0u, 0u};
      acc += qs[d] * ElemT<E>::chunk(raw, 0);
      acc += qs[d + 1] * ElemT<E>::chunk(raw, 1);
      acc += qs[d + 2] * ElemT<E>::chunk(raw, 2);
      acc += qs[d + 3] * ElemT<E>::chunk(raw, 3);
    }
  }
  return acc;
}

// One query row (b, h, r) of the per-row gather forward for any head_dim (a
// multiple of 4, up to 256), by one wave (the body of gather_fwd_kernel,
// esa_fwd_gather.hip, which describes it; also the band forward's path for
// rows whose positions are not consecutive): scratch is 384 floats of LDS
// private to the wave (q, the chunk's probabilities and keys).
template <Elem E, bool PATTERN>
__device__ __forceinline__ void gather_one_row_any(const GatherArgs& A, int b, int h, int r,
                                                   float* scratch, int lane) {
  using T = typename ElemT<E>::T;
  const int kvh = h / A.groups;
  const int D = A.D;
  float* qs = scratch;                // D <= 256 floats
  float* ps = scratch + 256;          // 64
  int* ks = (int*)(scratch + 320);    // 64

  const T* qrow = (const T*)A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)r * A.qss;
  for (int d = lane; d < D; d += 64) qs[d] = ElemT<E>::load(qrow + d);
  wave_sync_lds();

  const T* kbase = (const T*)A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh;
  const T* vbase = (const T*)A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh;
  RowEntries row;
  row.init<PATTERN>(A.src, h, r);

  float m = -INFINITY, l = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const int w = A.src.w;
  for (int c0 = 0; c0 < w; c0 += 64) {
    const int j = c0 + lane;
    bool valid = false;
    int64_t key = 0;
    if (j < w) row.entry<PATTERN>(A.src, h, r, j, valid, key);
    const bool in_range = key >= 0 && key < A.kv_len;
    float s = -INFINITY;
    if (valid) s = in_range ? row_dot<E>(qs, kbase + key * A.kss, D) * A.sm_scale : 0.f;
    const float cmax = wave_max(s);
    const float m_new = fmaxf(m, cmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float p = valid ? expf(s - m_use) : 0.f;
    const float alpha = expf(m - m_use);
    l = l * alpha + wave_sum(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] *= alpha;
    m = m_new;
    const float keep = j < w ? drop_factor(A.drop, b, h, r, j, A.H, A.q_len, w) : 0.f;
    ps[lane] = p * keep;
    ks[lane] = (valid && in_range) ? (int)key : -1;
    wave_sync_lds();
    const int nj = min(64, w - c0);
    for (int jj = 0; jj < nj; ++jj) {
      const float pj = ps[jj];
      const int kj = ks[jj];
      if (kj >= 0 && pj != 0.f) {
        const T* vr = vbase + (int64_t)kj * A.vss;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = lane + 64 * e;
          if (d < D) acc[e] += pj * ElemT<E>::load(vr + d);
        }
      }
    }
    wave_sync_lds();
  }

  const float inv = row.bad_pos ? __builtin_nanf("") : (l > 0.f ? 1.f / l : 0.f);
  T* orow = (T*)A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)r * A.oss;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int d = lane + 64 * e;
    if (d < D) ElemT<E>::store(orow + d, acc[e] * inv);
  }
  if (A.lse && lane == 0)
    A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + r] =
        row.bad_pos ? __builtin_nanf("") : (l > 0.f ? m + logf(l) : -INFINITY);
}

}  // namespace esa
