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

template <Elem E, bool PATTERN>
__global__ __launch_bounds__(256) void gather_fwd_kernel(GatherArgs A) {
  __shared__ float scratch_all[4][384];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = blockIdx.x * 4 + wave;
  const int h = blockIdx.y, b = blockIdx.z;
  if (r >= A.q_len) return;  // whole wave leaves; no block-level barrier below
  gather_one_row_any<E, PATTERN>(A, b, h, r, scratch_all[wave], lane);
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
  __shared__ float sc_all[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t wv = (int64_t)blockIdx.x * 4 + wave;
  // whole wave leaves; no block-level barrier below
  if (wv >= (int64_t)A.B * A.H * A.q_len) return;
  const int r = (int)(wv % A.q_len);
  const int h = (int)((wv / A.q_len) % A.H), b = (int)(wv / ((int64_t)A.q_len * A.H));
  gather_one_row<E, D, PATTERN>(A, b, h, r, sc_all[wave], lane);
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
