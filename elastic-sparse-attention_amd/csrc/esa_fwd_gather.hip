// Per-row gather forward (gfx950): one wave per (batch, head, query row).
//
// Two index sources share the kernel:
//   explicit  indices / mask arrays, the operator
//             ElasticSparseAttentionFunction.forward (elastic_sparse_attention.py:241-297)
//             with the Triton kernel's semantics (:117-166): a valid entry
//             whose index is outside [0, kv_len) scores 0 against zero K/V;
//             duplicates count once per entry.
//   pattern   each row's w indices regenerated on the device for query
//             position positions[r] (or r), masked entries set to 0 and
//             clamped to [0, kv_len - 1] as _triton_forward does (:602-615).
//
// Lanes split the row's entries 64 at a time for QK (each lane one key, a
// full dot product over D in float32), then split D for PV (each lane up to
// four d columns, one 64-key chunk at a time with p and the key broadcast
// through LDS).  Online softmax in float32 with accurate expf, so float32
// inputs meet a 1e-4 bound.
#include "esa_internal.hpp"

namespace esa {

template <typename T>
__device__ __forceinline__ float ld(const T* p);
template <>
__device__ __forceinline__ float ld<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float ld<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

template <typename T>
__device__ __forceinline__ void st(T* p, float v);
template <>
__device__ __forceinline__ void st<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void st<uint16_t>(uint16_t* p, float v) { *p = f32_to_bf16_bits(v); }

// dot(q, k_row) over D (D % 4 == 0); q in LDS as float.
template <typename T>
__device__ __forceinline__ float row_dot(const float* __restrict__ qs, const T* __restrict__ kr,
                                         int D);
template <>
__device__ __forceinline__ float row_dot<float>(const float* __restrict__ qs,
                                                const float* __restrict__ kr, int D) {
  float acc = 0.f;
  for (int d = 0; d < D; d += 4) {
    const f32x4 kv = *(const f32x4*)(kr + d);
    acc += qs[d] * kv[0];
    acc += qs[d + 1] * kv[1];
    acc += qs[d + 2] * kv[2];
    acc += qs[d + 3] * kv[3];
  }
  return acc;
}
template <>
__device__ __forceinline__ float row_dot<uint16_t>(const float* __restrict__ qs,
                                                   const uint16_t* __restrict__ kr, int D) {
  float acc = 0.f;
  for (int d = 0; d < D; d += 4) {
    const u32x2 kv = *(const u32x2*)(kr + d);
    acc += qs[d] * __uint_as_float(kv[0] << 16);
    acc += qs[d + 1] * __uint_as_float(kv[0] & 0xffff0000u);
    acc += qs[d + 2] * __uint_as_float(kv[1] << 16);
    acc += qs[d + 3] * __uint_as_float(kv[1] & 0xffff0000u);
  }
  return acc;
}

__device__ __forceinline__ int64_t load_int(const void* base, int bytes, int64_t off) {
  if (bytes == 8) return ((const int64_t*)base)[off];
  if (bytes == 4) return ((const int32_t*)base)[off];
  return ((const uint8_t*)base)[off];
}

template <typename T, bool PATTERN>
__global__ __launch_bounds__(256) void gather_fwd_kernel(GatherArgs A) {
  __shared__ float qs_all[4][256];
  __shared__ float ps_all[4][64];
  __shared__ int ks_all[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = blockIdx.x * 4 + wave;
  const int h = blockIdx.y, b = blockIdx.z;
  if (r >= A.q_len) return;  // whole wave leaves; no block-level barrier below
  const int kvh = h / A.groups;
  const int D = A.D;
  float* qs = qs_all[wave];
  float* ps = ps_all[wave];
  int* ks = ks_all[wave];

  const T* qrow = (const T*)A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)r * A.qss;
  for (int d = lane; d < D; d += 64) qs[d] = ld<T>(qrow + d);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  const T* kbase = (const T*)A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh;
  const T* vbase = (const T*)A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh;

  int pos = r;
  bool bad_pos = false;  // a position outside [0, kv_len): the row reads NaN
  HeadWeights hw{};
  RowParams rp{};
  if (PATTERN) {
    if (A.positions) {
      // negative positions count from the end, as torch indexing does
      const int64_t p0 = A.positions[r];
      const int64_t p64 = p0 < 0 ? p0 + A.kv_len : p0;
      bad_pos = p64 < 0 || p64 >= A.kv_len;
      pos = bad_pos ? 0 : (int)p64;
    }
    hw = head_weights(A.pc, h);
    rp = row_params(A.pc, pos);
  }

  float m = -INFINITY, l = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < A.w; c0 += 64) {
    const int j = c0 + lane;
    bool valid = false;
    int64_t key = 0;
    if (j < A.w) {
      if (PATTERN) {
        const int idx = interp_index(oversized(rp, j), oversized(rp, j + 1), hw);
        valid = idx <= pos;
        key = valid ? idx : 0;
        key = key < 0 ? 0 : (key > A.kv_len - 1 ? A.kv_len - 1 : key);
      } else {
        key = load_int(A.indices, A.index_bytes, (int64_t)h * A.ish + (int64_t)r * A.iss + j);
        valid = load_int(A.mask, A.mask_bytes, (int64_t)h * A.msh + (int64_t)r * A.mss + j) != 0;
      }
    }
    const bool in_range = key >= 0 && key < A.kv_len;
    float s = -INFINITY;
    if (valid) s = in_range ? row_dot<T>(qs, kbase + key * A.kss, D) * A.sm_scale : 0.f;
    const float cmax = wave_max(s);
    const float m_new = fmaxf(m, cmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float p = valid ? expf(s - m_use) : 0.f;
    const float alpha = expf(m - m_use);
    l = l * alpha + wave_sum(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] *= alpha;
    m = m_new;
    ps[lane] = p;
    ks[lane] = (valid && in_range) ? (int)key : -1;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int nj = min(64, A.w - c0);
    for (int jj = 0; jj < nj; ++jj) {
      const float pj = ps[jj];
      const int kj = ks[jj];
      if (kj >= 0 && pj != 0.f) {
        const T* vr = vbase + (int64_t)kj * A.vss;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = lane + 64 * e;
          if (d < D) acc[e] += pj * ld<T>(vr + d);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  const float inv = bad_pos ? __builtin_nanf("") : (l > 0.f ? 1.f / l : 0.f);
  T* orow = (T*)A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)r * A.oss;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int d = lane + 64 * e;
    if (d < D) st<T>(orow + d, acc[e] * inv);
  }
  if (A.lse && lane == 0)
    A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + r] =
        bad_pos ? __builtin_nanf("") : (l > 0.f ? m + logf(l) : -INFINITY);
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

// ---------------------------------------------------------------------------
// Cooperative-row variant for D = 64, 128, 256 with 16-byte aligned rows (the
// decode shapes): one wave per (batch, head, query row) as above, waves
// numbered over (batch, head, row) with the row fastest (a one-row decode
// step fills every wave of a block; a block per row would leave three of
// its four waves idle), but each
// K and V row is read by LPK = D * sizeof(T) / 16 lanes, 16 bytes each, so
// one load instruction covers KPI = 64 / LPK rows in whole cache lines, and a
// chunk's K and V rows (SK keys, NI = SK / KPI instructions each) are all in
// flight before the first score is formed.  Scores: each lane's 16-byte dot
// product, summed over the row's LPK lanes.  PV: each lane accumulates p * V
// over its 16 bytes of the rows it loaded; the KPI row groups are summed at
// the end.  Same online softmax, index semantics and float32 accuracy as
// gather_fwd_kernel (accurate expf; only the order of float32 additions
// differs).
template <typename T, int D, bool PATTERN>
__global__ __launch_bounds__(256, 2) void gather_rows_kernel(GatherArgs A) {
  constexpr int EPL = 16 / (int)sizeof(T);  // elements per lane per load
  constexpr int LPK = D / EPL;              // lanes per row
  constexpr int KPI = 64 / LPK;             // rows per load instruction
  constexpr int SK = 16 * KPI < 64 ? 16 * KPI : 64;  // keys per chunk
  constexpr int NI = SK / KPI;              // load instructions per chunk
  static_assert(LPK <= 64 && 64 % LPK == 0 && NI <= 16, "row split");
  __shared__ float sc_all[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t wv = (int64_t)blockIdx.x * 4 + wave;
  // whole wave leaves; no block-level barrier below
  if (wv >= (int64_t)A.B * A.H * A.q_len) return;
  const int r = (int)(wv % A.q_len);
  const int h = (int)((wv / A.q_len) % A.H), b = (int)(wv / ((int64_t)A.q_len * A.H));
  const int kvh = h / A.groups;
  float* sc = sc_all[wave];
  const int gk = lane / LPK;  // row of an instruction this lane loads
  const int ln = lane % LPK;  // its 16-byte piece: elements EPL ln .. + EPL

  float qv[EPL];
  {
    const T* qrow = (const T*)A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)r * A.qss;
    const u32x4 raw = *(const u32x4*)(qrow + EPL * ln);
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      if (sizeof(T) == 2)
        qv[e] = __uint_as_float((e & 1) ? (raw[e / 2] & 0xffff0000u) : (raw[e / 2] << 16));
      else
        qv[e] = __uint_as_float(raw[e]);
    }
  }
  const T* kbase = (const T*)A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh + EPL * ln;
  const T* vbase = (const T*)A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh + EPL * ln;

  int pos = r;
  bool bad_pos = false;  // a position outside [0, kv_len): the row reads NaN
  HeadWeights hw{};
  RowParams rp{};
  if (PATTERN) {
    if (A.positions) {
      // negative positions count from the end, as torch indexing does
      const int64_t p0 = A.positions[r];
      const int64_t p64 = p0 < 0 ? p0 + A.kv_len : p0;
      bad_pos = p64 < 0 || p64 >= A.kv_len;
      pos = bad_pos ? 0 : (int)p64;
    }
    hw = head_weights(A.pc, h);
    rp = row_params(A.pc, pos);
  }

  auto dot16 = [&](const u32x4& raw) {
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float x = sizeof(T) == 2
                          ? __uint_as_float((e & 1) ? (raw[e / 2] & 0xffff0000u) : (raw[e / 2] << 16))
                          : __uint_as_float(raw[e]);
      acc += qv[e] * x;
    }
    return acc;
  };

  float m = -INFINITY, l = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  for (int c0 = 0; c0 < A.w; c0 += SK) {
    // slot `lane` of the chunk: entry c0 + lane
    const int j = c0 + lane;
    bool valid = false;
    int64_t key = 0;
    if (lane < SK && j < A.w) {
      if (PATTERN) {
        const int idx = interp_index(oversized(rp, j), oversized(rp, j + 1), hw);
        valid = idx <= pos;
        key = valid ? idx : 0;
        key = key < 0 ? 0 : (key > A.kv_len - 1 ? A.kv_len - 1 : key);
      } else {
        key = load_int(A.indices, A.index_bytes, (int64_t)h * A.ish + (int64_t)r * A.iss + j);
        valid = load_int(A.mask, A.mask_bytes, (int64_t)h * A.msh + (int64_t)r * A.mss + j) != 0;
      }
    }
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
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < SK) sc[lane] = (valid && in_range) ? p : 0.f;  // PV weight of the slot
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int t = 0; t < NI; ++t) {
      const float pt = sc[KPI * t + gk];
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float x = sizeof(T) == 2 ? __uint_as_float((e & 1) ? (vd[t][e / 2] & 0xffff0000u)
                                                                  : (vd[t][e / 2] << 16))
                                       : __uint_as_float(vd[t][e]);
        acc[e] += pt * x;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // the KPI row groups' partial sums: lanes ln, ln + LPK, ...
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1)
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] += __shfl_xor(acc[e], off, 64);

  const float inv = bad_pos ? __builtin_nanf("") : (l > 0.f ? 1.f / l : 0.f);
  if (gk == 0) {
    T* orow = (T*)A.o + (int64_t)b * A.osb + (int64_t)h * A.osh + (int64_t)r * A.oss + EPL * ln;
    u32x4 w;
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      if (sizeof(T) == 2)
        w[e2] = (uint32_t)f32_to_bf16_bits(acc[2 * e2] * inv) |
                ((uint32_t)f32_to_bf16_bits(acc[2 * e2 + 1] * inv) << 16);
      else
        w[e2] = __float_as_uint(acc[e2] * inv);
    }
    *(u32x4*)orow = w;
  }
  if (A.lse && lane == 0)
    A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + r] =
        bad_pos ? __builtin_nanf("") : (l > 0.f ? m + logf(l) : -INFINITY);
}

// The cooperative kernel takes D = 64, 128, 256 and needs every Q, K, V and
// O row 16-byte aligned (bases and strides).
static bool rows_aligned16(const GatherArgs& a, int es) {
  if (a.D != 64 && a.D != 128 && a.D != 256) return false;
  const int64_t epl = 16 / es;
  const void* ptrs[] = {a.q, a.k, a.v, a.o};
  for (const void* p : ptrs)
    if (((uintptr_t)p & 15) != 0) return false;
  const int64_t st[] = {a.qsb, a.qsh, a.qss, a.ksb, a.ksh, a.kss,
                        a.vsb, a.vsh, a.vss, a.osb, a.osh, a.oss};
  for (int64_t x : st)
    if (x % epl != 0) return false;
  return true;
}

template <typename T, bool PATTERN>
static void launch_rows(const GatherArgs& a, dim3 grid, hipStream_t stream) {
  if (a.D == 64)
    gather_rows_kernel<T, 64, PATTERN><<<grid, 256, 0, stream>>>(a);
  else if (a.D == 128)
    gather_rows_kernel<T, 128, PATTERN><<<grid, 256, 0, stream>>>(a);
  else
    gather_rows_kernel<T, 256, PATTERN><<<grid, 256, 0, stream>>>(a);
}

hipError_t launch_gather_fwd(const GatherArgs& a, bool f32, bool pattern, hipStream_t stream) {
  if (a.q_len <= 0 || a.B <= 0 || a.H <= 0) return hipSuccess;
  dim3 grid((unsigned)((a.q_len + 3) / 4), (unsigned)a.H, (unsigned)a.B);
  // the cooperative kernel's one-dimensional grid: four waves per block,
  // within the 2^32 work-items of a dispatch
  const int64_t coop_blocks = ((int64_t)a.B * a.H * a.q_len + 3) / 4;
  if (rows_aligned16(a, f32 ? 4 : 2) && coop_blocks * 256 <= (int64_t)UINT32_MAX) {
    grid = dim3((unsigned)coop_blocks);
    if (f32) {
      if (pattern)
        launch_rows<float, true>(a, grid, stream);
      else
        launch_rows<float, false>(a, grid, stream);
    } else {
      if (pattern)
        launch_rows<uint16_t, true>(a, grid, stream);
      else
        launch_rows<uint16_t, false>(a, grid, stream);
    }
    return hipGetLastError();
  }
  if (f32) {
    if (pattern)
      gather_fwd_kernel<float, true><<<grid, 256, 0, stream>>>(a);
    else
      gather_fwd_kernel<float, false><<<grid, 256, 0, stream>>>(a);
  } else {
    if (pattern)
      gather_fwd_kernel<uint16_t, true><<<grid, 256, 0, stream>>>(a);
    else
      gather_fwd_kernel<uint16_t, false><<<grid, 256, 0, stream>>>(a);
  }
  return hipGetLastError();
}

}  // namespace esa
