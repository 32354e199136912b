// Per-row gather forward (gfx950): one wave per (batch, head, query row).
//
// Two index sources share the kernels (esa_gather.hpp):
//   explicit  indices / mask arrays, the operator
//             ElasticSparseAttentionFunction.forward (elastic_sparse_attention.py:241-297)
//             with the Triton kernel's semantics (:117-166): a valid entry
//             whose index is outside [0, kv_len) scores 0 against zero K/V;
//             duplicates count once per entry.
//   pattern   each row's w indices regenerated on the device for query
//             position positions[r] (or r), masked entries set to 0 and
//             clamped to [0, kv_len - 1] as _triton_forward does (:602-615).
//
// q, k, v and o are float32, bfloat16 or float16; everything is computed in
// float32 with accurate expf (float32 inputs meet a 1e-4 bound), and o is
// stored in the inputs' type.  With dropout (the naive path in training
// mode, :674) each probability is multiplied by its entry's keep factor in
// PV; the normaliser and lse stay those of the undropped probabilities, as
// torch.dropout after the softmax leaves them.
//
// gather_fwd_kernel: lanes split the row's entries 64 at a time for QK (each
// lane one key, a full dot product over D in float32), then split D for PV
// (each lane up to four d columns, one 64-key chunk at a time with p and the
// key broadcast through LDS).  gather_rows_kernel (D = 64, 128, 256 with
// 16-byte aligned rows) reads each K and V row with D * elem / 16 lanes.
// gather_weights_kernel writes the naive path's attention weights from the
// forward's lse.
#include "esa_gather.hpp"

namespace esa {

namespace {

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

template <Elem E, bool PATTERN>
__global__ __launch_bounds__(256) void gather_fwd_kernel(GatherArgs A) {
  using T = typename ElemT<E>::T;
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

// ---------------------------------------------------------------------------
// Cooperative-row variant for D = 64, 128, 256 with 16-byte aligned rows (the
// decode shapes): one wave per (batch, head, query row) as above, waves
// numbered over (batch, head, row) with the row fastest (a one-row decode
// step fills every wave of a block; a block per row would leave three of
// its four waves idle), but each
// K and V row is read by LPK = D * elem / 16 lanes, 16 bytes each, so one
// load instruction covers KPI = 64 / LPK rows in whole cache lines, and a
// chunk's K and V rows (SK keys, NI = SK / KPI instructions each) are all in
// flight before the first score is formed.  Scores: each lane's 16-byte dot
// product, summed over the row's LPK lanes.  PV: each lane accumulates p * V
// over its 16 bytes of the rows it loaded; the KPI row groups are summed at
// the end.  Same online softmax, index semantics and float32 accuracy as
// gather_fwd_kernel (accurate expf; only the order of float32 additions
// differs).
template <Elem E, int D, bool PATTERN>
__global__ __launch_bounds__(256, 2) void gather_rows_kernel(GatherArgs A) {
  using T = typename ElemT<E>::T;
  constexpr int EPL = ElemT<E>::kPerChunk;  // elements per lane per load
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

// ---------------------------------------------------------------------------
// The naive path's attention weights (elastic_sparse_attention.py:669-674):
// weights[b, h, r, j] = softmax over the row's valid entries, times the
// entry's dropout factor, 0 for a masked entry, in q's type.  One wave per
// (batch, head, row), lane j one entry, from the forward's lse (natural
// log): p_j = exp(s_j - lse).
template <Elem E, bool PATTERN>
__global__ __launch_bounds__(256) void gather_weights_kernel(GatherArgs A) {
  using T = typename ElemT<E>::T;
  __shared__ float qs_all[4][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = blockIdx.x * 4 + wave;
  const int h = blockIdx.y, b = blockIdx.z;
  if (r >= A.q_len) return;
  const int kvh = h / A.groups;
  const int D = A.D;
  float* qs = qs_all[wave];
  const T* qrow = (const T*)A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)r * A.qss;
  for (int d = lane; d < D; d += 64) qs[d] = ElemT<E>::load(qrow + d);
  wave_sync_lds();
  const T* kbase = (const T*)A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh;
  RowEntries row;
  row.init<PATTERN>(A.src, h, r);
  const float lse = A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + r];
  T* wrow = (T*)A.weights + (int64_t)b * A.wsb + (int64_t)h * A.wsh + (int64_t)r * A.wss;
  const int w = A.src.w;
  for (int c0 = 0; c0 < w; c0 += 64) {
    const int j = c0 + lane;
    if (j >= w) break;
    bool valid = false;
    int64_t key = 0;
    row.entry<PATTERN>(A.src, h, r, j, valid, key);
    const bool in_range = key >= 0 && key < A.kv_len;
    float p = 0.f;
    if (valid) {
      const float s = in_range ? row_dot<E>(qs, kbase + key * A.kss, D) * A.sm_scale : 0.f;
      p = expf(s - lse) * drop_factor(A.drop, b, h, r, j, A.H, A.q_len, w);
    }
    if (row.bad_pos) p = __builtin_nanf("");
    ElemT<E>::store(wrow + j, p);
  }
}

// The cooperative kernel takes D = 64, 128, 256 and needs every Q, K, V and
// O row 16-byte aligned (bases and strides).
bool rows_aligned16(const GatherArgs& a, int es) {
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

template <Elem E, bool PATTERN>
void launch_rows(const GatherArgs& a, dim3 grid, hipStream_t stream) {
  if (a.D == 64)
    gather_rows_kernel<E, 64, PATTERN><<<grid, 256, 0, stream>>>(a);
  else if (a.D == 128)
    gather_rows_kernel<E, 128, PATTERN><<<grid, 256, 0, stream>>>(a);
  else
    gather_rows_kernel<E, 256, PATTERN><<<grid, 256, 0, stream>>>(a);
}

template <Elem E>
void launch_gather_elem(const GatherArgs& a, bool pattern, hipStream_t stream) {
  dim3 grid((unsigned)((a.q_len + 3) / 4), (unsigned)a.H, (unsigned)a.B);
  // the cooperative kernel's one-dimensional grid: four waves per block,
  // within the 2^32 work-items of a dispatch
  const int64_t coop_blocks = ((int64_t)a.B * a.H * a.q_len + 3) / 4;
  if (rows_aligned16(a, ElemT<E>::kBytes) && coop_blocks * 256 <= (int64_t)UINT32_MAX) {
    grid = dim3((unsigned)coop_blocks);
    if (pattern)
      launch_rows<E, true>(a, grid, stream);
    else
      launch_rows<E, false>(a, grid, stream);
    return;
  }
  if (pattern)
    gather_fwd_kernel<E, true><<<grid, 256, 0, stream>>>(a);
  else
    gather_fwd_kernel<E, false><<<grid, 256, 0, stream>>>(a);
}

template <Elem E>
void launch_weights_elem(const GatherArgs& a, bool pattern, hipStream_t stream) {
  dim3 grid((unsigned)((a.q_len + 3) / 4), (unsigned)a.H, (unsigned)a.B);
  if (pattern)
    gather_weights_kernel<E, true><<<grid, 256, 0, stream>>>(a);
  else
    gather_weights_kernel<E, false><<<grid, 256, 0, stream>>>(a);
}

}  // namespace

hipError_t launch_gather_fwd(const GatherArgs& a, bool pattern, hipStream_t stream) {
  if (a.q_len <= 0 || a.B <= 0 || a.H <= 0) return hipSuccess;
  switch ((Elem)a.elem) {
    case Elem::f32: launch_gather_elem<Elem::f32>(a, pattern, stream); break;
    case Elem::bf16: launch_gather_elem<Elem::bf16>(a, pattern, stream); break;
    default: launch_gather_elem<Elem::f16>(a, pattern, stream); break;
  }
  return hipGetLastError();
}

hipError_t launch_gather_weights(const GatherArgs& a, bool pattern, hipStream_t stream) {
  if (a.q_len <= 0 || a.B <= 0 || a.H <= 0) return hipSuccess;
  switch ((Elem)a.elem) {
    case Elem::f32: launch_weights_elem<Elem::f32>(a, pattern, stream); break;
    case Elem::bf16: launch_weights_elem<Elem::bf16>(a, pattern, stream); break;
    default: launch_weights_elem<Elem::f16>(a, pattern, stream); break;
  }
  return hipGetLastError();
}

}  // namespace esa
