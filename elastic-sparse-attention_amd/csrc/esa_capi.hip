// C ABI of libesa.so: argument checks on the host, then kernel launches.
// Declarations and contracts: include/esa.h.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <numeric>
#include <vector>

#include "esa.h"
#include "esa_internal.hpp"

using namespace esa;

namespace {

constexpr int64_t kMaxSeqLen = int64_t(1) << 26;  // int32 work items and LDS bitmap bounds
constexpr int kMaxW = 1 << 16;

// The two scalars the reference's layout formula casts to float32
// (elastic_sparse_attention.py:488-496): alpha = layer_idx / max(nl - 1, 1)
// and w * (1 - alpha), both formed in double as Python does.
PatternConsts make_consts(const esa_pattern& p) {
  PatternConsts pc;
  const double denom = p.num_hidden_layers > 1 ? (double)(p.num_hidden_layers - 1) : 1.0;
  volatile double alpha = (double)p.layer_idx / denom;
  volatile double one_minus = 1.0 - alpha;
  volatile double cw = (double)p.attention_length * one_minus;
  pc.a = (float)alpha;
  pc.c = (float)cw;
  pc.w = p.attention_length;
  pc.H = p.num_heads;
  return pc;
}

esa_status check_pattern(const esa_pattern* p) {
  if (!p) return ESA_ERR_NULL;
  if (p->seq_len < 1 || p->seq_len > kMaxSeqLen) return ESA_ERR_SHAPE;
  if (p->attention_length < 1 || p->attention_length > kMaxW) return ESA_ERR_SHAPE;
  if (p->num_hidden_layers < 1 || p->num_heads < 1) return ESA_ERR_SHAPE;
  if (p->block_m < 1 || p->block_n < 1 || p->block_m > 4096 || p->block_n > 4096)
    return ESA_ERR_SHAPE;
  return ESA_OK;
}

LayoutDims dims_of(const esa_pattern& p) {
  LayoutDims d;
  d.seq_len = p.seq_len;
  d.bm = p.block_m;
  d.bn = p.block_n;
  d.nqb = (p.seq_len + p.block_m - 1) / p.block_m;
  d.nkb = (p.seq_len + p.block_n - 1) / p.block_n;
  d.nwords = (d.nkb + 31) / 32;
  return d;
}

// Upper bound on active tiles: block qb can only reach keys <= its last row
// (valid indices are causal), and holds at most rows * w entries.
int64_t max_tiles_of(const esa_pattern& p, const LayoutDims& d) {
  int64_t per_head = 0;
  for (int qb = 0; qb < d.nqb; ++qb) {
    const int64_t last = std::min<int64_t>(p.seq_len, (int64_t)(qb + 1) * p.block_m) - 1;
    const int64_t rows = last - (int64_t)qb * p.block_m + 1;
    per_head += std::min<int64_t>(last / p.block_n + 1, rows * p.attention_length);
  }
  return per_head * p.num_heads;
}

size_t workspace_of(const esa_pattern& p, const LayoutDims& d) {
  const int64_t rows = (int64_t)p.num_heads * d.nqb;
  return (size_t)(rows * d.nwords * 4 + rows * 4 + 256);
}

bool aligned(const void* ptr, size_t a) { return ((uintptr_t)ptr % a) == 0; }

size_t elem_bytes(esa_dtype t) { return t == ESA_F32 ? 4 : 2; }

// rows rows of `stride` 16-bit elements span less than 2 GiB (the kernels'
// 32-bit buffer offsets); the stride is bounded first, so the product cannot
// overflow for any argument (rows <= kMaxSeqLen + 128)
bool span_fits_2g(int64_t rows, int64_t stride) {
  return stride >= 0 && stride < (int64_t(1) << 31) && rows * stride * 2 < (int64_t(1) << 31);
}

esa_status check_fwd_common(const esa_fwd_args* a) {
  if (!a || !a->q || !a->k || !a->v || !a->o) return ESA_ERR_NULL;
  if (a->dtype != ESA_F32 && a->dtype != ESA_BF16 && a->dtype != ESA_F16) return ESA_ERR_DTYPE;
  if (a->batch < 0 || a->num_heads < 1 || a->num_kv_heads < 1 || a->q_len < 0 || a->kv_len < 1 ||
      a->head_dim < 1)
    return ESA_ERR_SHAPE;
  if (a->num_heads % a->num_kv_heads != 0) return ESA_ERR_SHAPE;
  if (a->kv_len > kMaxSeqLen || a->q_len > kMaxSeqLen) return ESA_ERR_SHAPE;
  return ESA_OK;
}

GatherArgs gather_args_of(const esa_fwd_args* a) {
  GatherArgs g{};
  g.q = a->q; g.k = a->k; g.v = a->v; g.o = a->o; g.lse = a->lse;
  g.qsb = a->q_stride_b; g.qsh = a->q_stride_h; g.qss = a->q_stride_s;
  g.ksb = a->k_stride_b; g.ksh = a->k_stride_h; g.kss = a->k_stride_s;
  g.vsb = a->v_stride_b; g.vsh = a->v_stride_h; g.vss = a->v_stride_s;
  g.osb = a->o_stride_b; g.osh = a->o_stride_h; g.oss = a->o_stride_s;
  g.lsb = a->lse_stride_b; g.lsh = a->lse_stride_h;
  g.B = a->batch; g.H = a->num_heads; g.groups = a->num_heads / a->num_kv_heads;
  g.q_len = a->q_len; g.kv_len = a->kv_len; g.D = a->head_dim;
  g.sm_scale = a->sm_scale;
  g.elem = a->dtype;  // ESA_F32 / ESA_BF16 / ESA_F16 are Elem's codes
  g.src.kv_len = a->kv_len;
  return g;
}

esa_status check_gather_layout(const esa_fwd_args* a) {
  if (a->head_dim % 4 != 0 || a->head_dim > 256) return ESA_ERR_UNSUPPORTED;
  const size_t es = elem_bytes(a->dtype);
  // K rows are read 4 elements at a time.
  if (!aligned(a->k, 4 * es) || a->k_stride_s % 4 != 0 || a->k_stride_h % 4 != 0 ||
      a->k_stride_b % 4 != 0)
    return ESA_ERR_ALIGN;
  return ESA_OK;
}

// Work lists of the block-sparse kernels, laid out for the 8 XCDs of MI355X.
//
// Consecutive workgroup ids are dispatched round-robin over the XCDs
// (id % 8), and each XCD has its own L2.  Items come in streams (all query
// blocks of one (batch, head) for the forward; all key blocks of one
// (batch, kv head) for the backward's dK/dV), each walked from its last item
// to its first (the costliest first: later blocks see longer prefixes).
// The walk is cut into 8 runs of equal cost; run x goes to grid slots x,
// x + 8, x + 16, ..., so one XCD works through one or two streams' K/V (or
// Q/dO) at a time, their tiles staying in its L2, and ends on the cheapest
// items of its last stream.  Runs shorter than the longest are padded with
// -1 (an empty workgroup).
template <typename Cost, typename Id>
void plan_xcd_runs(int64_t streams, int per_stream, Cost cost, Id id, std::vector<int32_t>& grid) {
  constexpr int kXcd = 8;
  int64_t total = 0;
  for (int64_t st = 0; st < streams; ++st)
    for (int j = 0; j < per_stream; ++j) total += cost(st, j);
  const int64_t n = streams * per_stream;
  std::vector<std::vector<int32_t>> runs(kXcd);
  int64_t cum = 0;
  int x = 0;
  for (int64_t st = 0; st < streams; ++st) {
    for (int j = per_stream - 1; j >= 0; --j) {
      // move on once this run holds its share of the cost (by item count
      // when every item is free)
      while (x < kXcd - 1 && (total > 0 ? cum * kXcd >= (int64_t)(x + 1) * total
                                        : (int64_t)runs[x].size() * kXcd >= n))
        ++x;
      runs[x].push_back(id(st, j));
      cum += cost(st, j);
    }
  }
  size_t len = 0;
  for (auto& r : runs) len = std::max(len, r.size());
  grid.assign(len * kXcd, -1);
  for (int r = 0; r < kXcd; ++r)
    for (size_t i = 0; i < runs[r].size(); ++i) grid[i * kXcd + r] = runs[r][i];
}

// Forward: streams (b, h), items qb < nq, cost = active tiles.
void plan_xcd_grid(const int32_t* row_ptr, int nqb, int nq, int batch, int H,
                   std::vector<int32_t>& grid) {
  plan_xcd_runs(
      (int64_t)batch * H, nq,
      [&](int64_t st, int qb) {
        const int64_t row = (st % H) * nqb + qb;
        return (int64_t)(row_ptr[row + 1] - row_ptr[row]);
      },
      [&](int64_t st, int qb) { return (int32_t)(st * nqb + qb); }, grid);
}

esa_status hip_status(hipError_t e) { return e == hipSuccess ? ESA_OK : ESA_ERR_HIP; }

// Byte offsets of the gather backward's workspace regions (each 256-byte
// aligned): per batch element and entry a dV and a dK coefficient, two
// (key, entry id) pair buffers for the sort, the per-key segment starts and
// the sort's digit histograms, their scan and its chunk sums.
struct GatherBwdLayout {
  int64_t E;  // entries per batch element: H * q_len * w
  size_t cp, cs, ka, va, kb, vb, seg, hist, offs, parts, total;
};

esa_status gather_bwd_layout(const esa_bwd_args* a, int32_t w, GatherBwdLayout* L) {
  if (a->batch < 0 || a->num_heads < 1 || a->num_kv_heads < 1 || a->q_len < 0 || a->kv_len < 1 ||
      a->head_dim < 1 || w < 1 || w > kMaxW)
    return ESA_ERR_SHAPE;
  const int64_t E = (int64_t)a->num_heads * a->q_len * w;
  // entry ids and sorted positions are 32-bit; the sort keys' sentinel is
  // Hkv * kv_len
  if (E >= INT32_MAX || (int64_t)a->num_kv_heads * a->kv_len >= INT32_MAX) return ESA_ERR_SHAPE;
  int64_t hist_ints = 0, part_ints = 0;
  gather_bwd_sort_sizes(E, &hist_ints, &part_ints);
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t off = at;
    at += up(bytes);
    return off;
  };
  L->E = E;
  L->cp = take((size_t)a->batch * E * 4);
  L->cs = take((size_t)a->batch * E * 4);
  L->ka = take((size_t)E * 4);
  L->va = take((size_t)E * 4);
  L->kb = take((size_t)E * 4);
  L->vb = take((size_t)E * 4);
  L->seg = take(((size_t)a->num_kv_heads * a->kv_len + 1) * 4);
  L->hist = take((size_t)hist_ints * 4);
  L->offs = take((size_t)hist_ints * 4);
  L->parts = take((size_t)part_ints * 4);
  L->total = at;
  return ESA_OK;
}

// Checks shared by the gather backward entry points; fills g.
esa_status gather_bwd_args(const esa_bwd_args* a, int32_t w, void* workspace,
                           size_t workspace_bytes, GatherBwdArgs* g) {
  if (!a || !a->q || !a->k || !a->v || !a->o || !a->dout || !a->dq || !a->dk || !a->dv || !a->lse)
    return ESA_ERR_NULL;
  if (a->dtype != ESA_F32 && a->dtype != ESA_BF16 && a->dtype != ESA_F16) return ESA_ERR_DTYPE;
  if (a->num_heads < 1 || a->num_kv_heads < 1 || a->num_heads % a->num_kv_heads != 0)
    return ESA_ERR_SHAPE;
  if (a->kv_len > kMaxSeqLen || a->q_len > kMaxSeqLen) return ESA_ERR_SHAPE;
  if (a->head_dim % 4 != 0 || a->head_dim > 256) return ESA_ERR_UNSUPPORTED;
  GatherBwdLayout L;
  esa_status s = gather_bwd_layout(a, w, &L);
  if (s != ESA_OK) return s;
  // K and V rows are read 4 elements at a time
  const size_t es = elem_bytes(a->dtype);
  if (!aligned(a->k, 4 * es) || !aligned(a->v, 4 * es)) return ESA_ERR_ALIGN;
  const int64_t st[] = {a->k_stride_b, a->k_stride_h, a->k_stride_s,
                        a->v_stride_b, a->v_stride_h, a->v_stride_s};
  for (int64_t x : st)
    if (x % 4 != 0) return ESA_ERR_ALIGN;
  if (a->batch == 0) {  // nothing to write
    g->B = 0;
    return ESA_OK;
  }
  // (q_len = 0 still writes dK = dV = 0, as the reference's zeros_like does)
  if (!workspace) return ESA_ERR_NULL;
  if (workspace_bytes < L.total) return ESA_ERR_CAPACITY;
  if (!aligned(workspace, 256)) return ESA_ERR_ALIGN;
  GatherBwdArgs& t = *g;
  t = GatherBwdArgs{};
  t.q = a->q; t.k = a->k; t.v = a->v; t.o = a->o; t.dout = a->dout;
  t.dq = a->dq; t.dk = a->dk; t.dv = a->dv; t.lse = a->lse;
  t.qsb = a->q_stride_b; t.qsh = a->q_stride_h; t.qss = a->q_stride_s;
  t.ksb = a->k_stride_b; t.ksh = a->k_stride_h; t.kss = a->k_stride_s;
  t.vsb = a->v_stride_b; t.vsh = a->v_stride_h; t.vss = a->v_stride_s;
  t.osb = a->o_stride_b; t.osh = a->o_stride_h; t.oss = a->o_stride_s;
  t.dosb = a->dout_stride_b; t.dosh = a->dout_stride_h; t.doss = a->dout_stride_s;
  t.dqsb = a->dq_stride_b; t.dqsh = a->dq_stride_h; t.dqss = a->dq_stride_s;
  t.dksb = a->dk_stride_b; t.dksh = a->dk_stride_h; t.dkss = a->dk_stride_s;
  t.dvsb = a->dv_stride_b; t.dvsh = a->dv_stride_h; t.dvss = a->dv_stride_s;
  t.lsb = a->lse_stride_b; t.lsh = a->lse_stride_h;
  t.B = a->batch; t.H = a->num_heads; t.Hkv = a->num_kv_heads;
  t.groups = a->num_heads / a->num_kv_heads;
  t.q_len = a->q_len; t.kv_len = a->kv_len; t.D = a->head_dim;
  t.sm_scale = a->sm_scale;
  t.elem = a->dtype;
  t.src.w = w;
  t.src.kv_len = a->kv_len;
  t.drop.p = 0.f;
  t.drop.scale = 1.f;
  t.E = L.E;
  char* ws = (char*)workspace;
  t.cp = (float*)(ws + L.cp);
  t.cs = (float*)(ws + L.cs);
  t.keys_in = (uint32_t*)(ws + L.ka);
  t.vals_in = (uint32_t*)(ws + L.va);
  t.keys_out = (uint32_t*)(ws + L.kb);
  t.vals_out = (uint32_t*)(ws + L.vb);
  t.seg = (int32_t*)(ws + L.seg);
  t.hist = (int32_t*)(ws + L.hist);
  t.offs = (int32_t*)(ws + L.offs);
  t.parts = (int32_t*)(ws + L.parts);
  int bits = 1;
  while (bits < 32 && ((uint64_t)1 << bits) <= (uint64_t)a->num_kv_heads * a->kv_len) ++bits;
  t.key_bits = bits;  // the sentinel Hkv * kv_len fits
  return ESA_OK;
}

// Row stride of the backward's per-row workspace (delta, lse2): q_len rounded
// up to 32, plus 32, so a 32-row step that starts on a valid row reads inside
// its (b, h) rows
int bwd_qpad(int q_len) { return (q_len + 31) / 32 * 32 + 32; }

}  // namespace

extern "C" {

const char* esa_status_string(esa_status s) {
  switch (s) {
    case ESA_OK: return "ok";
    case ESA_ERR_NULL: return "null pointer";
    case ESA_ERR_SHAPE: return "invalid or inconsistent shape";
    case ESA_ERR_DTYPE: return "unsupported dtype";
    case ESA_ERR_ALIGN: return "misaligned pointer or stride";
    case ESA_ERR_UNSUPPORTED: return "unsupported configuration";
    case ESA_ERR_CAPACITY: return "buffer too small";
    case ESA_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

const char* esa_version(void) { return "esa-gfx950 0.1.0"; }

esa_status esa_layout_sizes(const esa_pattern* p, int32_t* num_qblocks, int32_t* num_kblocks,
                            int64_t* max_tiles, size_t* workspace_bytes) {
  esa_status s = check_pattern(p);
  if (s != ESA_OK) return s;
  const LayoutDims d = dims_of(*p);
  if ((int64_t)d.nwords * 4 > 65536) return ESA_ERR_SHAPE;  // LDS bitmap bound
  // row_ptr, the builder's scan and every tile id are int32
  if (max_tiles_of(*p, d) > INT32_MAX) return ESA_ERR_SHAPE;
  if (num_qblocks) *num_qblocks = d.nqb;
  if (num_kblocks) *num_kblocks = d.nkb;
  if (max_tiles) *max_tiles = max_tiles_of(*p, d);
  if (workspace_bytes) *workspace_bytes = workspace_of(*p, d);
  return ESA_OK;
}

esa_status esa_build_indices(const esa_pattern* p, int32_t row0, int32_t nrows, void* indices,
                             void* mask, int32_t elem_bytes, void* stream) {
  esa_status s = check_pattern(p);
  if (s != ESA_OK) return s;
  if (elem_bytes != 4 && elem_bytes != 8) return ESA_ERR_DTYPE;
  if (row0 < 0 || nrows < 0 || (int64_t)row0 + nrows > p->seq_len) return ESA_ERR_SHAPE;
  if (!indices && !mask) return ESA_OK;
  if (nrows == 0) return ESA_OK;
  if ((int64_t)nrows * p->attention_length > (int64_t(1) << 40)) return ESA_ERR_SHAPE;
  return hip_status(launch_indices(make_consts(*p), row0, nrows, indices, mask, elem_bytes,
                                   (hipStream_t)stream));
}

esa_status esa_build_dense_mask(const esa_pattern* p, int32_t row0, int32_t nrows,
                                int32_t ncols, uint8_t* mask, int64_t stride_h,
                                int64_t stride_s, void* stream) {
  esa_status s = check_pattern(p);
  if (s != ESA_OK) return s;
  if (!mask) return ESA_ERR_NULL;
  if (row0 < 0 || nrows < 0 || (int64_t)row0 + nrows > p->seq_len || ncols < 1)
    return ESA_ERR_SHAPE;
  if (p->num_heads > 65535) return ESA_ERR_UNSUPPORTED;  // grid.y
  // a row's bytes and the rows / heads must not overlap
  if (stride_s < ncols || (p->num_heads > 1 && stride_h < (int64_t)nrows * stride_s))
    return ESA_ERR_SHAPE;
  if (nrows == 0) return ESA_OK;
  return hip_status(launch_dense_mask(make_consts(*p), row0, nrows, ncols, mask, stride_h,
                                      stride_s, (hipStream_t)stream));
}

esa_status esa_build_layout(const esa_pattern* p, int32_t* row_ptr, int32_t* col_idx,
                            int64_t col_capacity, void* workspace, size_t workspace_bytes,
                            void* stream) {
  esa_status s = check_pattern(p);
  if (s != ESA_OK) return s;
  if (!row_ptr || !col_idx || !workspace) return ESA_ERR_NULL;
  const LayoutDims d = dims_of(*p);
  if ((int64_t)d.nwords * 4 > 65536) return ESA_ERR_SHAPE;
  if (max_tiles_of(*p, d) > INT32_MAX) return ESA_ERR_SHAPE;
  if (col_capacity < max_tiles_of(*p, d)) return ESA_ERR_CAPACITY;
  if (workspace_bytes < workspace_of(*p, d)) return ESA_ERR_CAPACITY;
  if (!aligned(workspace, 4)) return ESA_ERR_ALIGN;
  return hip_status(
      launch_layout(make_consts(*p), d, row_ptr, col_idx, workspace, (hipStream_t)stream));
}

esa_status esa_plan_schedule(const esa_pattern* p, const int32_t* row_ptr_host, int32_t q_len,
                             int32_t batch, int32_t* items_host, int64_t items_capacity,
                             int64_t* num_items) {
  esa_status s = check_pattern(p);
  if (s != ESA_OK) return s;
  if (!row_ptr_host || !num_items) return ESA_ERR_NULL;
  if (q_len < 0 || q_len > p->seq_len || batch < 0) return ESA_ERR_SHAPE;
  const LayoutDims d = dims_of(*p);
  if ((int64_t)batch * p->num_heads * d.nqb > INT32_MAX) return ESA_ERR_SHAPE;
  const int nq = (q_len + p->block_m - 1) / p->block_m;
  const int64_t n = (int64_t)batch * p->num_heads * nq;
  std::vector<int32_t> grid;
  plan_xcd_grid(row_ptr_host, d.nqb, nq, batch, p->num_heads, grid);
  *num_items = (int64_t)grid.size();
  if (!items_host) return ESA_OK;  // size query
  if (items_capacity < (int64_t)grid.size()) return ESA_ERR_CAPACITY;
  std::copy(grid.begin(), grid.end(), items_host);
  (void)n;
  return ESA_OK;
}

esa_status esa_elastic_fwd(const esa_fwd_args* a, const esa_pattern* p, const int32_t* row_ptr,
                           const int32_t* col_idx, const int32_t* row_ptr_host,
                           const uint32_t* stage_masks, int64_t stage_mask_words,
                           const int32_t* items, int64_t num_items, void* stream) {
  esa_status s = check_fwd_common(a);
  if (s != ESA_OK) return s;
  s = check_pattern(p);
  if (s != ESA_OK) return s;
  if (!row_ptr || !col_idx || !items) return ESA_ERR_NULL;
  if (a->dtype != ESA_BF16 && a->dtype != ESA_F16) return ESA_ERR_DTYPE;
  if (a->head_dim != 64 && a->head_dim != 128) return ESA_ERR_UNSUPPORTED;
  // 128-row query blocks with key blocks of 128 (two 64-key stages each) or
  // 64 keys; or 64-row query blocks with 32-key blocks
  const bool rows64 = p->block_m == 64 && p->block_n == 32;
  if (!rows64 && (p->block_m != 128 || (p->block_n != 128 && p->block_n != 64)))
    return ESA_ERR_UNSUPPORTED;
  // stage masks exist for layouts whose key blocks are the stages
  if (stage_masks && p->block_n == 128) return ESA_ERR_UNSUPPORTED;
  if (stage_masks && !aligned(stage_masks, 8)) return ESA_ERR_ALIGN;
  if (stage_masks) {
    // the kernel reads the masks of every tile of the layout it walks: the
    // buffer must hold them all (sized from the host copy of row_ptr)
    if (!row_ptr_host) return ESA_ERR_NULL;
    int64_t need = 0;
    s = esa_stage_masks_size(p, row_ptr_host, &need);
    if (s != ESA_OK) return s;
    if (stage_mask_words < need) return ESA_ERR_CAPACITY;
  }
  // The per-tile key masks assume strictly rising indices, which holds for
  // 0 <= alpha <= 1.
  if (p->layer_idx < 0 || p->layer_idx > std::max(p->num_hidden_layers - 1, 0))
    return ESA_ERR_UNSUPPORTED;
  if (p->num_heads != a->num_heads) return ESA_ERR_SHAPE;
  if (a->q_len > a->kv_len || a->q_len > p->seq_len) return ESA_ERR_SHAPE;
  // the kernel folds the key mask into the scaled score as -inf
  if (!(a->sm_scale > 0.f) || !std::isfinite(a->sm_scale)) return ESA_ERR_UNSUPPORTED;
  // K/V rows are addressed through 32-bit buffer offsets per (batch, kv head)
  // (rows up to one tile past kv_len are addressed, and read as zeros)
  if (!span_fits_2g((int64_t)a->kv_len + 128, a->k_stride_s) ||
      !span_fits_2g((int64_t)a->kv_len + 128, a->v_stride_s) || a->k_stride_s < a->head_dim ||
      a->v_stride_s < a->head_dim)
    return ESA_ERR_UNSUPPORTED;
  const LayoutDims d = dims_of(*p);
  const int nq = (a->q_len + p->block_m - 1) / p->block_m;
  // a plan from esa_plan_schedule holds every item once plus at most 7 pads
  // per item slot row
  const int64_t n_real = (int64_t)a->batch * a->num_heads * nq;
  if (num_items < n_real || num_items > 8 * std::max<int64_t>(n_real, 1)) return ESA_ERR_SHAPE;
  // 16-byte row loads and 8-byte output stores.
  if (!aligned(a->q, 16) || !aligned(a->k, 16) || !aligned(a->v, 16) || !aligned(a->o, 8))
    return ESA_ERR_ALIGN;
  const int64_t st[] = {a->q_stride_b, a->q_stride_h, a->q_stride_s, a->k_stride_b,
                        a->k_stride_h, a->k_stride_s, a->v_stride_b, a->v_stride_h,
                        a->v_stride_s};
  for (int64_t x : st)
    if (x % 8 != 0) return ESA_ERR_ALIGN;
  if (a->o_stride_b % 4 || a->o_stride_h % 4 || a->o_stride_s % 4) return ESA_ERR_ALIGN;
  if (num_items == 0 || a->batch == 0 || a->q_len == 0) return ESA_OK;

  TileArgs t{};
  t.q = (const uint16_t*)a->q; t.k = (const uint16_t*)a->k; t.v = (const uint16_t*)a->v;
  t.o = (uint16_t*)a->o; t.lse = a->lse;
  t.qsb = a->q_stride_b; t.qsh = a->q_stride_h; t.qss = a->q_stride_s;
  t.ksb = a->k_stride_b; t.ksh = a->k_stride_h; t.kss = a->k_stride_s;
  t.vsb = a->v_stride_b; t.vsh = a->v_stride_h; t.vss = a->v_stride_s;
  t.osb = a->o_stride_b; t.osh = a->o_stride_h; t.oss = a->o_stride_s;
  t.lsb = a->lse_stride_b; t.lsh = a->lse_stride_h;
  t.H = a->num_heads; t.groups = a->num_heads / a->num_kv_heads;
  t.q_len = a->q_len; t.kv_len = a->kv_len; t.nqb = d.nqb; t.nq = nq;
  t.num_bh = a->batch * a->num_heads;
  t.stage_shift = p->block_n == 128 ? 1 : 0;
  t.rows64 = rows64 ? 1 : 0;
  t.scale_log2 = a->sm_scale * 1.4426950408889634f;
  t.pc = make_consts(*p);
  t.row_ptr = row_ptr; t.col_idx = col_idx; t.items = items;
  t.smask = stage_masks;
  t.elem = a->dtype;
  return hip_status(launch_tile_fwd(t, a->head_dim, num_items, (hipStream_t)stream));
}

}  // extern "C"

namespace {

// Checks and arguments of the band-gathered forward (16 query rows per
// group; a band's buffer offsets reach up to 16 rows past kv_len).
esa_status band_args_of(const esa_fwd_args* a, const esa_pattern* p, const int64_t* positions,
                        BandArgs* out) {
  constexpr int rows_per_item = 16, pad_rows = 16;
  esa_status s = check_fwd_common(a);
  if (s != ESA_OK) return s;
  s = check_pattern(p);
  if (s != ESA_OK) return s;
  if (a->dtype != ESA_BF16 && a->dtype != ESA_F16) return ESA_ERR_DTYPE;
  // kernels at D = 64, 128 and 256; a head_dim between them (a multiple of
  // 8: whole 16-byte chunks) runs the next one up with zero padding
  if (a->head_dim < 8 || a->head_dim > 256 || a->head_dim % 8 != 0) return ESA_ERR_UNSUPPORTED;
  // one wave holds a row's band descriptors for at most 64 bands; indices
  // rise with the band (0 <= alpha <= 1)
  if (p->attention_length > 64) return ESA_ERR_UNSUPPORTED;
  if (p->layer_idx < 0 || p->layer_idx > std::max(p->num_hidden_layers - 1, 0))
    return ESA_ERR_UNSUPPORTED;
  if (p->num_heads != a->num_heads) return ESA_ERR_SHAPE;
  // (with positions the rows may be any positions, as esa_elastic_fwd_rows
  // takes them)
  if (!positions && (a->q_len > a->kv_len || a->q_len > p->seq_len)) return ESA_ERR_SHAPE;
  if (!(a->sm_scale > 0.f) || !std::isfinite(a->sm_scale)) return ESA_ERR_UNSUPPORTED;
  // band descriptors pack the first key in 24 bits; K/V rows are addressed
  // through 32-bit buffer offsets per (batch, kv head)
  if (a->kv_len >= (1 << 24)) return ESA_ERR_UNSUPPORTED;
  if (!span_fits_2g((int64_t)a->kv_len + pad_rows, a->k_stride_s) ||
      !span_fits_2g((int64_t)a->kv_len + pad_rows, a->v_stride_s) ||
      a->k_stride_s < a->head_dim || a->v_stride_s < a->head_dim)
    return ESA_ERR_UNSUPPORTED;
  // 16-byte row loads and stores
  if (!aligned(a->q, 16) || !aligned(a->k, 16) || !aligned(a->v, 16) || !aligned(a->o, 16))
    return ESA_ERR_ALIGN;
  const int64_t st[] = {a->q_stride_b, a->q_stride_h, a->q_stride_s, a->k_stride_b,
                        a->k_stride_h, a->k_stride_s, a->v_stride_b, a->v_stride_h,
                        a->v_stride_s, a->o_stride_b, a->o_stride_h, a->o_stride_s};
  for (int64_t x : st)
    if (x % 8 != 0) return ESA_ERR_ALIGN;
  BandArgs& t = *out;
  t = BandArgs{};
  if (a->batch == 0 || a->q_len == 0) return ESA_OK;
  const int ng = (a->q_len + rows_per_item - 1) / rows_per_item;
  const int64_t n_groups = (int64_t)a->batch * a->num_heads * ng;
  if (n_groups > INT32_MAX / 2) return ESA_ERR_SHAPE;
  t.q = (const uint16_t*)a->q; t.k = (const uint16_t*)a->k; t.v = (const uint16_t*)a->v;
  t.o = (uint16_t*)a->o; t.lse = a->lse;
  t.qsb = a->q_stride_b; t.qsh = a->q_stride_h; t.qss = a->q_stride_s;
  t.ksb = a->k_stride_b; t.ksh = a->k_stride_h; t.kss = a->k_stride_s;
  t.vsb = a->v_stride_b; t.vsh = a->v_stride_h; t.vss = a->v_stride_s;
  t.osb = a->o_stride_b; t.osh = a->o_stride_h; t.oss = a->o_stride_s;
  t.lsb = a->lse_stride_b; t.lsh = a->lse_stride_h;
  t.H = a->num_heads; t.groups = a->num_heads / a->num_kv_heads; t.q_len = a->q_len;
  t.ng = ng;
  t.n_groups = (int)n_groups;
  t.per_xcd = (int)((n_groups + 7) / 8);
  t.scale_log2 = a->sm_scale * 1.4426950408889634f;
  t.pc = make_consts(*p);
  t.elem = a->dtype;
  t.positions = positions;
  t.kv_len = a->kv_len;
  t.sm_scale = a->sm_scale;
  t.d_real = a->head_dim;
  return ESA_OK;
}

}  // namespace

extern "C" {

esa_status esa_elastic_fwd_band(const esa_fwd_args* a, const esa_pattern* p,
                                const int64_t* positions, void* stream) {
  BandArgs t;
  esa_status s = band_args_of(a, p, positions, &t);
  if (s != ESA_OK || t.n_groups == 0) return s;
  return hip_status(launch_band_fwd(t, a->head_dim, (hipStream_t)stream));
}

esa_status esa_elastic_fwd_rows(const esa_fwd_args* a, const esa_pattern* p,
                                const int64_t* positions, void* stream) {
  esa_status s = check_fwd_common(a);
  if (s != ESA_OK) return s;
  s = check_pattern(p);
  if (s != ESA_OK) return s;
  if (p->num_heads != a->num_heads) return ESA_ERR_SHAPE;
  if (!positions && a->q_len > a->kv_len) return ESA_ERR_SHAPE;
  s = check_gather_layout(a);
  if (s != ESA_OK) return s;
  GatherArgs g = gather_args_of(a);
  g.src.w = p->attention_length;
  g.src.pc = make_consts(*p);
  g.src.positions = positions;
  return hip_status(launch_gather_fwd(g, true, (hipStream_t)stream));
}

esa_status esa_elastic_fwd_naive(const esa_fwd_args* a, const esa_pattern* p,
                                 const int64_t* positions, const esa_naive_opts* opts,
                                 void* stream) {
  esa_status s = check_fwd_common(a);
  if (s != ESA_OK) return s;
  s = check_pattern(p);
  if (s != ESA_OK) return s;
  if (!opts) return ESA_ERR_NULL;
  if (p->num_heads != a->num_heads) return ESA_ERR_SHAPE;
  if (!positions && a->q_len > a->kv_len) return ESA_ERR_SHAPE;
  if (!(opts->dropout_p >= 0.f && opts->dropout_p < 1.f)) return ESA_ERR_SHAPE;
  // the weights are formed from the forward's log-sum-exp
  if (opts->weights && !a->lse) return ESA_ERR_NULL;
  s = check_gather_layout(a);
  if (s != ESA_OK) return s;
  GatherArgs g = gather_args_of(a);
  g.src.w = p->attention_length;
  g.src.pc = make_consts(*p);
  g.src.positions = positions;
  g.drop.p = opts->dropout_p;
  g.drop.scale = opts->dropout_p > 0.f ? 1.0f / (1.0f - opts->dropout_p) : 1.0f;
  g.drop.seed = opts->seed;
  g.weights = opts->weights;
  g.wsb = opts->weights_stride_b; g.wsh = opts->weights_stride_h; g.wss = opts->weights_stride_s;
  hipError_t e = launch_gather_fwd(g, true, (hipStream_t)stream);
  if (e == hipSuccess && opts->weights) e = launch_gather_weights(g, true, (hipStream_t)stream);
  return hip_status(e);
}

esa_status esa_sparse_fwd(const esa_fwd_args* a, const void* indices, int32_t index_bytes,
                          int64_t idx_stride_h, int64_t idx_stride_s, const void* mask,
                          int32_t mask_bytes, int64_t mask_stride_h, int64_t mask_stride_s,
                          int32_t attn_length, void* stream) {
  esa_status s = check_fwd_common(a);
  if (s != ESA_OK) return s;
  if (!indices || !mask) return ESA_ERR_NULL;
  if (index_bytes != 4 && index_bytes != 8) return ESA_ERR_DTYPE;
  if (mask_bytes != 1 && mask_bytes != 4 && mask_bytes != 8) return ESA_ERR_DTYPE;
  if (attn_length < 1 || attn_length > kMaxW) return ESA_ERR_SHAPE;
  s = check_gather_layout(a);
  if (s != ESA_OK) return s;
  GatherArgs g = gather_args_of(a);
  g.src.w = attn_length;
  g.src.indices = indices; g.src.mask = mask;
  g.src.index_bytes = index_bytes; g.src.mask_bytes = mask_bytes;
  g.src.ish = idx_stride_h; g.src.iss = idx_stride_s;
  g.src.msh = mask_stride_h; g.src.mss = mask_stride_s;
  return hip_status(launch_gather_fwd(g, false, (hipStream_t)stream));
}

esa_status esa_plan_bwd(const esa_pattern* p, const int32_t* row_ptr_host,
                        const int32_t* col_idx_host, int32_t q_len, int32_t batch,
                        int32_t num_kv_heads, int32_t* tile_row, int32_t* kv_ptr,
                        int32_t* kv_tiles, int64_t kv_tiles_capacity, int32_t* kv_items,
                        int64_t kv_items_capacity, int64_t* num_kv_tiles,
                        int64_t* num_kv_items) {
  esa_status s = check_pattern(p);
  if (s != ESA_OK) return s;
  if (!row_ptr_host || !col_idx_host || !num_kv_tiles || !num_kv_items) return ESA_ERR_NULL;
  if (q_len < 0 || q_len > p->seq_len || batch < 0 || num_kv_heads < 1 ||
      p->num_heads % num_kv_heads != 0)
    return ESA_ERR_SHAPE;
  const LayoutDims d = dims_of(*p);
  const int H = p->num_heads, groups = H / num_kv_heads;
  const int nq = (q_len + p->block_m - 1) / p->block_m;
  if ((int64_t)batch * num_kv_heads * d.nkb > INT32_MAX) return ESA_ERR_SHAPE;
  // tiles per (kv head, key block) over query blocks below nq
  const int64_t nrow = (int64_t)num_kv_heads * d.nkb;
  std::vector<int64_t> cnt(nrow + 1, 0);
  for (int h = 0; h < H; ++h)
    for (int qb = 0; qb < nq; ++qb)
      for (int32_t t = row_ptr_host[(int64_t)h * d.nqb + qb]; t < row_ptr_host[(int64_t)h * d.nqb + qb + 1]; ++t)
        ++cnt[(int64_t)(h / groups) * d.nkb + col_idx_host[t] + 1];
  for (int64_t r = 0; r < nrow; ++r) cnt[r + 1] += cnt[r];
  const int64_t ntiles = cnt[nrow];
  std::vector<int32_t> grid;
  plan_xcd_runs(
      (int64_t)batch * num_kv_heads, d.nkb,
      [&](int64_t st, int kb) {
        const int64_t r = (st % num_kv_heads) * d.nkb + kb;
        return cnt[r + 1] - cnt[r];
      },
      [&](int64_t st, int kb) { return (int32_t)(st * d.nkb + kb); }, grid);
  *num_kv_tiles = ntiles;
  *num_kv_items = (int64_t)grid.size();
  if (!tile_row || !kv_ptr || !kv_tiles || !kv_items) return ESA_OK;  // size query
  if (kv_tiles_capacity < ntiles || kv_items_capacity < (int64_t)grid.size())
    return ESA_ERR_CAPACITY;
  for (int h = 0; h < H; ++h)
    for (int qb = 0; qb < d.nqb; ++qb)
      for (int32_t t = row_ptr_host[(int64_t)h * d.nqb + qb]; t < row_ptr_host[(int64_t)h * d.nqb + qb + 1]; ++t)
        tile_row[t] = h * d.nqb + qb;
  std::vector<int64_t> fill(cnt.begin(), cnt.end() - 1);
  for (int h = 0; h < H; ++h)
    for (int qb = 0; qb < nq; ++qb)
      for (int32_t t = row_ptr_host[(int64_t)h * d.nqb + qb]; t < row_ptr_host[(int64_t)h * d.nqb + qb + 1]; ++t)
        kv_tiles[fill[(int64_t)(h / groups) * d.nkb + col_idx_host[t]]++] = t;
  for (int64_t r = 0; r <= nrow; ++r) kv_ptr[r] = (int32_t)cnt[r];
  std::copy(grid.begin(), grid.end(), kv_items);
  return ESA_OK;
}

esa_status esa_build_tile_masks(const esa_pattern* p, const int32_t* row_ptr,
                                const int32_t* col_idx, const int32_t* row_ptr_host,
                                int32_t q_len, uint32_t* mask_t, int64_t mask_capacity,
                                void* stream) {
  esa_status s = check_pattern(p);
  if (s != ESA_OK) return s;
  if (!row_ptr || !col_idx || !row_ptr_host || !mask_t) return ESA_ERR_NULL;
  if (p->block_m != 128 || p->block_n != 128) return ESA_ERR_UNSUPPORTED;
  if (q_len < 0 || q_len > p->seq_len) return ESA_ERR_SHAPE;
  const LayoutDims d = dims_of(*p);
  if (q_len == 0) return ESA_OK;
  // the masks of the tiles of query blocks below ceil(q_len / 128) are
  // written; the last head's end among them bounds every tile id written
  const int nq = (q_len + p->block_m - 1) / p->block_m;
  const int64_t need = (int64_t)row_ptr_host[(int64_t)(p->num_heads - 1) * d.nqb + nq];
  if (need < 0 || mask_capacity < need * 512) return ESA_ERR_CAPACITY;
  if (!aligned(mask_t, 4)) return ESA_ERR_ALIGN;
  return hip_status(launch_tile_masks(make_consts(*p), row_ptr, col_idx, d.nqb, q_len, mask_t,
                                      (hipStream_t)stream));
}

esa_status esa_stage_masks_size(const esa_pattern* p, const int32_t* row_ptr_host,
                                int64_t* words) {
  if (!p || !row_ptr_host || !words) return ESA_ERR_NULL;
  esa_status s = check_pattern(p);
  if (s != ESA_OK) return s;
  const bool ok = (p->block_m == 64 && p->block_n == 32) ||
                  (p->block_m == 128 && (p->block_n == 64 || p->block_n == 128));
  if (!ok) return ESA_ERR_UNSUPPORTED;
  const LayoutDims d = dims_of(*p);
  const int64_t tiles = row_ptr_host[(int64_t)p->num_heads * d.nqb];
  if (tiles < 0) return ESA_ERR_SHAPE;
  *words = tiles * p->block_m * (p->block_n / 32);
  return ESA_OK;
}

esa_status esa_build_stage_masks(const esa_pattern* p, const int32_t* row_ptr,
                                 const int32_t* col_idx, const int32_t* row_ptr_host,
                                 uint32_t* masks, int64_t capacity_words, void* stream) {
  int64_t need = 0;
  esa_status s = esa_stage_masks_size(p, row_ptr_host, &need);
  if (s != ESA_OK) return s;
  if (!row_ptr || !col_idx || !masks) return ESA_ERR_NULL;
  if (p->layer_idx < 0 || p->layer_idx > std::max(p->num_hidden_layers - 1, 0))
    return ESA_ERR_UNSUPPORTED;
  if (capacity_words < need) return ESA_ERR_CAPACITY;
  if (!aligned(masks, 8)) return ESA_ERR_ALIGN;
  if (need == 0) return ESA_OK;
  return hip_status(launch_stage_masks(make_consts(*p), dims_of(*p), row_ptr, col_idx, masks,
                                       (hipStream_t)stream));
}

// The band dK/dV's split at the last layer of a pattern (alpha = 1): entry 0
// of a query head with interpolation weight t has key ~ t (i + 1) / w, so the
// heads with small t put a key of each of the first blocks into about
// 16 w / t rows, and every row's entry 0 into block 0 for t = 0.  Key block
// 0 of every (b, kv head) (about groups * q_len / 32 steps against a mean of
// about groups * w steps) is split over split_parts waves of about 200
// steps each.  Measured at B=1 H=32 L=32768 D=128: with 8 kv heads the last
// layer's backward takes 7.64 ms unsplit, 5.30 ms with block 0 split and
// 5.47 ms with blocks 0 .. 7 split (the other heavy blocks stay under a
// slot's share); with 32 kv heads all three are within 1.5%.
int bwd_split_parts(const esa_bwd_args* a) {
  const int groups = a->num_kv_heads > 0 ? a->num_heads / a->num_kv_heads : 1;
  const int64_t p = ((int64_t)groups * a->q_len + 6143) / 6144;
  return (int)std::min<int64_t>(std::max<int64_t>(p, 1), 32);
}
int bwd_split_blocks(const esa_bwd_args*) { return 1; }

// Byte offsets of the MFMA backward's workspace regions: delta and lse2 per
// row (rows of each (b, h) padded to qpad, bwd_qpad), the split dK / dV's
// float32 partial sums and arrival counters (when it splits), then the
// non-finite flags (one byte per 16-row dQ group and per 16-key dK / dV
// block), 256-byte aligned; the total is a multiple of 256 bytes.
struct BwdWsLayout {
  size_t part_buf, part_cnt, flags, total;
  int64_t n_qflags, n_kvflags;
};

static BwdWsLayout bwd_ws_layout(const esa_bwd_args* a) {
  BwdWsLayout L{};
  size_t bytes = (size_t)2 * a->batch * a->num_heads * bwd_qpad(a->q_len) * sizeof(float);
  L.part_buf = L.part_cnt = bytes;
  const int parts = bwd_split_parts(a);
  if (parts > 1) {
    const size_t n_split = (size_t)a->batch * a->num_kv_heads * bwd_split_blocks(a);
    bytes += n_split * parts * 2 * 16 * a->head_dim * sizeof(float);
    L.part_cnt = bytes;
    bytes += (n_split * sizeof(int) + 15) / 16 * 16;
  }
  L.flags = (bytes + 255) / 256 * 256;
  L.n_qflags = (int64_t)a->batch * a->num_heads * ((a->q_len + 15) / 16);
  L.n_kvflags = (int64_t)a->batch * a->num_kv_heads * ((std::max(a->kv_len, 0) + 15) / 16);
  L.total = (L.flags + (size_t)(L.n_qflags + L.n_kvflags) + 255) / 256 * 256;
  return L;
}

esa_status esa_bwd_workspace_size(const esa_bwd_args* a, size_t* workspace_bytes) {
  if (!a || !workspace_bytes) return ESA_ERR_NULL;
  if (a->batch < 0 || a->num_heads < 1 || a->num_kv_heads < 1 || a->q_len < 0 ||
      a->head_dim < 1)
    return ESA_ERR_SHAPE;
  *workspace_bytes = bwd_ws_layout(a).total;
  return ESA_OK;
}

}  // extern "C"

namespace {

// Workspace of esa_elastic_bwd_noalloc: one array per device, set up by the
// code-object loader when the library's kernels are loaded on that device and
// held until the process ends.  Host code never passes `scratch` itself (on
// the host the name is a stand-in, not a device address): the device address
// comes from hipGetSymbolAddress, once per device, in scratch_of.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Looks up `scratch`'s device address on device dev once (with dev
// current; the caller's device is restored) and keeps it.  esa_init_device
// calls this at set-up, outside any graph capture; a call of the entry point
// on a device nobody initialised does it on its first call.
esa_status scratch_on(int dev, void** out = nullptr) {
  if (dev < 0 || dev >= kMaxDevices) return ESA_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return ESA_ERR_HIP;
    if (dev != cur && hipSetDevice(dev) != hipSuccess) return ESA_ERR_HIP;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (dev != cur && hipSetDevice(cur) != hipSuccess) return ESA_ERR_HIP;
    if (e != hipSuccess || !ptr) return ESA_ERR_HIP;
    g_scratch_ptr[dev] = ptr;
  }
  if (out) *out = g_scratch_ptr[dev];
  return ESA_OK;
}

// Device address of `scratch` on the device `stream` belongs to.
esa_status scratch_of(hipStream_t stream, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return ESA_ERR_HIP;
  if (stream && hipStreamGetDevice(stream, &dev) != hipSuccess) return ESA_ERR_HIP;
  return scratch_on(dev, out);
}

// The backward's argument checks and launches; `workspace` is the caller's
// buffer (esa_elastic_bwd) or the device's scratch array
// (esa_elastic_bwd_noalloc, workspace NULL until the checks pass).
esa_status elastic_bwd_impl(const esa_bwd_args* a, const esa_pattern* p, const int32_t* row_ptr,
                            const int32_t* col_idx, const int32_t* row_ptr_host,
                            const int32_t* q_items, int64_t num_q_items,
                            const int32_t* tile_row, const int32_t* kv_ptr,
                            const int32_t* kv_tiles, const int32_t* kv_items,
                            int64_t num_kv_items, const uint32_t* mask_t, int64_t mask_t_words,
                            const uint32_t* q_masks, int64_t q_mask_words, void* workspace,
                            size_t workspace_bytes, bool static_ws, void* stream) {
  if (!a || !a->q || !a->k || !a->v || !a->o || !a->dout || !a->dq || !a->dk || !a->dv || !a->lse)
    return ESA_ERR_NULL;
  esa_status s = check_pattern(p);
  if (s != ESA_OK) return s;
  // q_items NULL: dQ by the band-gathered kernel (no work list or layout);
  // kv_items NULL: dK / dV by the band-gathered kernel (no work list, tile
  // lists or masks)
  const bool band_dq = q_items == nullptr, band_dkdv = kv_items == nullptr;
  if ((!static_ws && !workspace) || (!band_dq && (!row_ptr || !col_idx)) ||
      (!band_dkdv && (!tile_row || !kv_ptr || !kv_tiles || !mask_t)))
    return ESA_ERR_NULL;
  if ((band_dq || band_dkdv) && (p->attention_length > 64 || a->kv_len >= (1 << 24)))
    return ESA_ERR_UNSUPPORTED;
  if (a->dtype != ESA_BF16 && a->dtype != ESA_F16) return ESA_ERR_DTYPE;
  if (a->batch < 0 || a->num_heads < 1 || a->num_kv_heads < 1 || a->q_len < 0 || a->kv_len < 1 ||
      a->num_heads % a->num_kv_heads != 0 || a->num_heads != p->num_heads)
    return ESA_ERR_SHAPE;
  if (a->head_dim != 64 && a->head_dim != 128) return ESA_ERR_UNSUPPORTED;
  if (p->block_m != 128 || p->block_n != 128) return ESA_ERR_UNSUPPORTED;
  if (p->layer_idx < 0 || p->layer_idx > std::max(p->num_hidden_layers - 1, 0))
    return ESA_ERR_UNSUPPORTED;
  if (a->q_len > a->kv_len || a->q_len > p->seq_len || a->kv_len > kMaxSeqLen) return ESA_ERR_SHAPE;
  // the block-sparse dK/dV writes the key blocks of the pattern's seq_len only
  if (!band_dkdv && a->kv_len > p->seq_len) return ESA_ERR_SHAPE;
  if (!(a->sm_scale > 0.f) || !std::isfinite(a->sm_scale)) return ESA_ERR_UNSUPPORTED;
  // (rows up to one tile past the length are addressed, and read as zeros)
  if (!span_fits_2g((int64_t)a->kv_len + 128, a->k_stride_s) ||
      !span_fits_2g((int64_t)a->kv_len + 128, a->v_stride_s) ||
      !span_fits_2g((int64_t)a->q_len + 128, a->q_stride_s) ||
      !span_fits_2g((int64_t)a->q_len + 128, a->dout_stride_s) || a->q_stride_s < a->head_dim ||
      a->dout_stride_s < a->head_dim || a->k_stride_s < a->head_dim || a->v_stride_s < a->head_dim)
    return ESA_ERR_UNSUPPORTED;
  const void* ptrs[] = {a->q, a->k, a->v, a->o, a->dout, a->dq, a->dk, a->dv};
  for (const void* x : ptrs)
    if (!aligned(x, 16)) return ESA_ERR_ALIGN;
  const int64_t st[] = {a->q_stride_b,  a->q_stride_h,  a->q_stride_s,  a->k_stride_b,
                        a->k_stride_h,  a->k_stride_s,  a->v_stride_b,  a->v_stride_h,
                        a->v_stride_s,  a->o_stride_b,  a->o_stride_h,  a->o_stride_s,
                        a->dout_stride_b, a->dout_stride_h, a->dout_stride_s, a->dq_stride_b,
                        a->dq_stride_h, a->dq_stride_s, a->dk_stride_b, a->dk_stride_h,
                        a->dk_stride_s, a->dv_stride_b, a->dv_stride_h, a->dv_stride_s};
  for (int64_t x : st)
    if (x % 8 != 0) return ESA_ERR_ALIGN;
  size_t need = 0;
  esa_bwd_workspace_size(a, &need);
  if (workspace_bytes < need) return ESA_ERR_CAPACITY;
  if (!static_ws && !aligned(workspace, 16)) return ESA_ERR_ALIGN;
  // row masks serve the block-sparse dQ only (16-byte loads)
  if (q_masks && band_dq) return ESA_ERR_UNSUPPORTED;
  if (q_masks && !aligned(q_masks, 16)) return ESA_ERR_ALIGN;
  const LayoutDims d = dims_of(*p);
  const int nq = (a->q_len + 127) / 128;
  // the masks are read by tile id: each buffer must hold every tile the
  // kernels reach, sized from the host copy of row_ptr
  if ((q_masks || !band_dkdv) && !row_ptr_host) return ESA_ERR_NULL;
  if (q_masks) {
    int64_t need = 0;
    s = esa_stage_masks_size(p, row_ptr_host, &need);
    if (s != ESA_OK) return s;
    if (q_mask_words < need) return ESA_ERR_CAPACITY;
  }
  if (!band_dkdv) {
    const int64_t tiles = row_ptr_host[(int64_t)(p->num_heads - 1) * d.nqb + nq];
    if (tiles < 0) return ESA_ERR_SHAPE;
    if (mask_t_words < tiles * 512) return ESA_ERR_CAPACITY;
  }
  const int64_t n_real = (int64_t)a->batch * a->num_heads * nq;
  if (!band_dq && (num_q_items < n_real || num_q_items > 8 * std::max<int64_t>(n_real, 1)))
    return ESA_ERR_SHAPE;
  const int64_t kv_real = (int64_t)a->batch * a->num_kv_heads * d.nkb;
  if (!band_dkdv &&
      (num_kv_items < kv_real || num_kv_items > 8 * std::max<int64_t>(kv_real, 1)))
    return ESA_ERR_SHAPE;
  if (a->batch == 0 || a->q_len == 0) return ESA_OK;
  if (static_ws) {
    esa_status ss = scratch_of((hipStream_t)stream, &workspace);
    if (ss != ESA_OK) return ss;
  }

  BwdArgs t{};
  t.q = (const uint16_t*)a->q; t.k = (const uint16_t*)a->k; t.v = (const uint16_t*)a->v;
  t.o = (const uint16_t*)a->o; t.dout = (const uint16_t*)a->dout;
  t.dq = (uint16_t*)a->dq; t.dk = (uint16_t*)a->dk; t.dv = (uint16_t*)a->dv;
  t.lse = a->lse; t.delta = (float*)workspace; t.mask_t = mask_t; t.qmask = q_masks;
  t.qsb = a->q_stride_b; t.qsh = a->q_stride_h; t.qss = a->q_stride_s;
  t.ksb = a->k_stride_b; t.ksh = a->k_stride_h; t.kss = a->k_stride_s;
  t.vsb = a->v_stride_b; t.vsh = a->v_stride_h; t.vss = a->v_stride_s;
  t.osb = a->o_stride_b; t.osh = a->o_stride_h; t.oss = a->o_stride_s;
  t.dosb = a->dout_stride_b; t.dosh = a->dout_stride_h; t.doss = a->dout_stride_s;
  t.dqsb = a->dq_stride_b; t.dqsh = a->dq_stride_h; t.dqss = a->dq_stride_s;
  t.dksb = a->dk_stride_b; t.dksh = a->dk_stride_h; t.dkss = a->dk_stride_s;
  t.dvsb = a->dv_stride_b; t.dvsh = a->dv_stride_h; t.dvss = a->dv_stride_s;
  t.lsb = a->lse_stride_b; t.lsh = a->lse_stride_h;
  t.B = a->batch; t.H = a->num_heads; t.Hkv = a->num_kv_heads;
  t.groups = a->num_heads / a->num_kv_heads;
  t.q_len = a->q_len; t.kv_len = a->kv_len;
  t.qpad = bwd_qpad(a->q_len);
  t.nqb = d.nqb; t.nq = nq; t.nkb = d.nkb;
  t.sm_scale = a->sm_scale; t.scale_log2 = a->sm_scale * 1.4426950408889634f;
  t.pc = make_consts(*p);
  t.elem = a->dtype;
  t.row_ptr = row_ptr; t.col_idx = col_idx; t.q_items = q_items;
  t.tile_row = tile_row; t.kv_ptr = kv_ptr; t.kv_tiles = kv_tiles; t.kv_items = kv_items;
  t.ng = (a->q_len + 15) / 16;
  const int64_t n_groups = (int64_t)a->batch * a->num_heads * t.ng;
  if (band_dq && n_groups > INT32_MAX / 2) return ESA_ERR_SHAPE;
  t.n_groups = (int)n_groups;
  t.per_xcd = (int)((n_groups + 7) / 8);
  t.nkb16 = (a->kv_len + 15) / 16;
  const int64_t n_kblk = (int64_t)a->batch * a->num_kv_heads * t.nkb16;
  if (band_dkdv && n_kblk > INT32_MAX / 2) return ESA_ERR_SHAPE;
  // (the band dK/dV reaches lse2 from a delta row by a 32-bit buffer offset)
  if (band_dkdv && (int64_t)a->batch * a->num_heads * t.qpad * 8 >= (int64_t(1) << 31))
    return ESA_ERR_UNSUPPORTED;
  t.n_kblk = (int)n_kblk;
  t.kchunk = ((int64_t)a->batch * a->num_kv_heads) % 8 == 0 ? (int)(n_kblk / 8) : 8;
  t.split_parts = 1;
  t.split_blocks = 0;
  t.n_bkv = a->batch * a->num_kv_heads;
  if (band_dkdv && t.pc.a == 1.0f && bwd_split_parts(a) > 1) {
    t.split_parts = bwd_split_parts(a);
    t.split_blocks = bwd_split_blocks(a);
    const int64_t n_split = (int64_t)t.n_bkv * t.split_blocks;
    if (n_split * (t.split_parts - 1) > INT32_MAX / 2) return ESA_ERR_SHAPE;
    t.n_extra = (int)((n_split * (t.split_parts - 1) + 7) / 8 * 8);
  }
  const BwdWsLayout wl = bwd_ws_layout(a);
  t.part_buf = (float*)((char*)workspace + wl.part_buf);
  t.part_cnt = (int*)((char*)workspace + wl.part_cnt);
  t.flags = (uint8_t*)workspace + wl.flags;
  if (wl.n_qflags + wl.n_kvflags > INT32_MAX / 2) return ESA_ERR_SHAPE;
  t.n_qflags = (int)wl.n_qflags;
  t.n_kvflags = (int)wl.n_kvflags;
  return hip_status(launch_tile_bwd(t, a->head_dim, band_dq ? -1 : num_q_items,
                                    band_dkdv ? -1 : num_kv_items, (hipStream_t)stream));
}

}  // namespace

extern "C" {

esa_status esa_elastic_bwd(const esa_bwd_args* a, const esa_pattern* p, const int32_t* row_ptr,
                           const int32_t* col_idx, const int32_t* row_ptr_host,
                           const int32_t* q_items, int64_t num_q_items,
                           const int32_t* tile_row, const int32_t* kv_ptr,
                           const int32_t* kv_tiles, const int32_t* kv_items,
                           int64_t num_kv_items, const uint32_t* mask_t, int64_t mask_t_words,
                           const uint32_t* q_masks, int64_t q_mask_words, void* workspace,
                           size_t workspace_bytes, void* stream) {
  return elastic_bwd_impl(a, p, row_ptr, col_idx, row_ptr_host, q_items, num_q_items, tile_row,
                          kv_ptr, kv_tiles, kv_items, num_kv_items, mask_t, mask_t_words,
                          q_masks, q_mask_words, workspace, workspace_bytes, false, stream);
}

size_t esa_bwd_noalloc_max_workspace(void) { return kScratchBytes; }

esa_status esa_elastic_bwd_noalloc(const esa_bwd_args* a, const esa_pattern* p,
                                   const int32_t* row_ptr, const int32_t* col_idx,
                                   const int32_t* row_ptr_host, const int32_t* q_items,
                                   int64_t num_q_items, const int32_t* tile_row,
                                   const int32_t* kv_ptr, const int32_t* kv_tiles,
                                   const int32_t* kv_items, int64_t num_kv_items,
                                   const uint32_t* mask_t, int64_t mask_t_words,
                                   const uint32_t* q_masks, int64_t q_mask_words,
                                   void* stream) {
  return elastic_bwd_impl(a, p, row_ptr, col_idx, row_ptr_host, q_items, num_q_items, tile_row,
                          kv_ptr, kv_tiles, kv_items, num_kv_items, mask_t, mask_t_words,
                          q_masks, q_mask_words, nullptr, kScratchBytes, true, stream);
}

esa_status esa_init_device(int32_t device) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) return ESA_ERR_HIP;
  if (device < 0 || device >= count) return ESA_ERR_SHAPE;
  return scratch_on(device);
}

esa_status esa_gather_bwd_workspace_size(const esa_bwd_args* a, int32_t attn_length,
                                         size_t* workspace_bytes) {
  if (!a || !workspace_bytes) return ESA_ERR_NULL;
  GatherBwdLayout L;
  esa_status s = gather_bwd_layout(a, attn_length, &L);
  if (s != ESA_OK) return s;
  *workspace_bytes = L.total;
  return ESA_OK;
}

esa_status esa_sparse_bwd(const esa_bwd_args* a, const void* indices, int32_t index_bytes,
                          int64_t idx_stride_h, int64_t idx_stride_s, const void* mask,
                          int32_t mask_bytes, int64_t mask_stride_h, int64_t mask_stride_s,
                          int32_t attn_length, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (!indices || !mask) return ESA_ERR_NULL;
  if (index_bytes != 4 && index_bytes != 8) return ESA_ERR_DTYPE;
  if (mask_bytes != 1 && mask_bytes != 4 && mask_bytes != 8) return ESA_ERR_DTYPE;
  GatherBwdArgs g;
  esa_status s = gather_bwd_args(a, attn_length, workspace, workspace_bytes, &g);
  if (s != ESA_OK || g.B == 0) return s;
  g.src.indices = indices; g.src.mask = mask;
  g.src.index_bytes = index_bytes; g.src.mask_bytes = mask_bytes;
  g.src.ish = idx_stride_h; g.src.iss = idx_stride_s;
  g.src.msh = mask_stride_h; g.src.mss = mask_stride_s;
  return hip_status(launch_gather_bwd(g, false, (hipStream_t)stream));
}

esa_status esa_elastic_bwd_rows(const esa_bwd_args* a, const esa_pattern* p,
                                const int64_t* positions, float dropout_p, uint64_t seed,
                                void* workspace, size_t workspace_bytes, void* stream) {
  esa_status s = check_pattern(p);
  if (s != ESA_OK) return s;
  if (!a) return ESA_ERR_NULL;
  if (p->num_heads != a->num_heads) return ESA_ERR_SHAPE;
  if (!positions && a->q_len > a->kv_len) return ESA_ERR_SHAPE;
  if (!(dropout_p >= 0.f && dropout_p < 1.f)) return ESA_ERR_SHAPE;
  GatherBwdArgs g;
  s = gather_bwd_args(a, p->attention_length, workspace, workspace_bytes, &g);
  if (s != ESA_OK || g.B == 0) return s;
  g.src.pc = make_consts(*p);
  g.src.positions = positions;
  g.drop.p = dropout_p;
  g.drop.scale = dropout_p > 0.f ? 1.0f / (1.0f - dropout_p) : 1.0f;
  g.drop.seed = seed;
  return hip_status(launch_gather_bwd(g, true, (hipStream_t)stream));
}

esa_status esa_reachability(int32_t seq_len, int32_t attention_length,
                            int32_t num_hidden_layers, int32_t num_heads, int32_t position,
                            uint32_t* reach, uint32_t* work, int32_t* layer_counts,
                            void* stream) {
  if (!reach || !work) return ESA_ERR_NULL;
  if (reach == work) return ESA_ERR_SHAPE;
  esa_pattern p{};
  p.seq_len = seq_len;
  p.attention_length = attention_length;
  p.num_hidden_layers = num_hidden_layers;
  p.num_heads = num_heads;
  p.block_m = p.block_n = 128;
  esa_status st = check_pattern(&p);
  if (st != ESA_OK) return st;
  if (position < 0 || position >= seq_len) return ESA_ERR_SHAPE;
  if (!aligned(reach, 4) || !aligned(work, 4) || !aligned(layer_counts, 4)) return ESA_ERR_ALIGN;
  // layers in processing order: the last layer first
  std::vector<PatternConsts> layers((size_t)num_hidden_layers);
  for (int k = 0; k < num_hidden_layers; ++k) {
    p.layer_idx = num_hidden_layers - 1 - k;
    layers[(size_t)k] = make_consts(p);
  }
  return hip_status(launch_reachability(layers.data(), num_hidden_layers, position, reach, work,
                                        layer_counts, (hipStream_t)stream));
}

}  // extern "C"
