// Internal declarations shared by the kernels and the C-ABI layer.
#pragma once
#include "esa_common.hpp"

namespace esa {

struct LayoutDims {
  int seq_len, bm, bn;
  int nqb;     // query blocks per head
  int nkb;     // key tiles
  int nwords;  // 32-bit words per tile bitmap
};

// Arguments of the block-sparse MFMA forward.
struct TileArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t qsb, qsh, qss;
  int64_t ksb, ksh, kss;
  int64_t vsb, vsh, vss;
  int64_t osb, osh, oss;
  int64_t lsb, lsh;
  int H, groups, q_len, kv_len;
  int nqb;     // query blocks per head in the layout
  int nq;      // query blocks a q_len-row forward visits (<= nqb)
  int num_bh;  // batch * H
  int stage_shift;  // layout key blocks are (stage keys) << stage_shift keys
  int rows64;       // 1: 64-row items (2 waves) over a 64 x 32 layout
  int elem;         // Elem of q, k, v, o: bf16 or f16
  float scale_log2;  // sm_scale * log2(e)
  PatternConsts pc;
  const int32_t* row_ptr;
  const int32_t* col_idx;
  const int32_t* items;
  // per-stage row masks from esa_build_stage_masks (stage layouts only), or
  // nullptr: the kernel walks each row's index list itself
  const uint32_t* smask;
};

// Arguments of the band-gathered forward (prefill rows 0 .. q_len - 1).
struct BandArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t qsb, qsh, qss;
  int64_t ksb, ksh, kss;
  int64_t vsb, vsh, vss;
  int64_t osb, osh, oss;
  int64_t lsb, lsh;
  int H, groups, q_len;
  int ng;        // 16-row groups per (batch, head)
  int n_groups;  // batch * H * ng
  int per_xcd;   // groups per XCD range
  float scale_log2;  // sm_scale * log2(e)
  PatternConsts pc;
  int elem;      // Elem of q, k, v, o: bf16 or f16
  // query positions (cache_position): row r is position positions[r] (a
  // negative one counting from kv_len), or r when NULL
  const int64_t* positions;
  int kv_len;
  float sm_scale;
  // the inputs' head_dim (a multiple of 8) when it is below the kernel's D:
  // dims d_real .. D - 1 of Q, K and V read as zeros and O's are not stored
  int d_real;
  // entry rotation of the band forward, in 64ths of an entry per group
  // dispatched on an XCD (set by launch_band_fwd from the grid's size)
  int rot_rate;
};

// Where a query row's w entries come from: the elastic pattern (regenerated
// on the device, rows at positions[r] or r) or explicit index / mask arrays
// [H, q_len, w].
struct IndexSource {
  int w;       // entries per row
  int kv_len;  // keys; pattern keys are clamped to [0, kv_len - 1]
  // pattern source
  PatternConsts pc;
  const int64_t* positions;  // may be NULL (row r is position r)
  // explicit-index source
  const void* indices;
  const void* mask;
  int index_bytes, mask_bytes;
  int64_t ish, iss, msh, mss;
};

// Attention dropout on the probabilities (the naive path in training mode,
// elastic_sparse_attention.py:674): p = 0 switches it off.
struct DropoutArgs {
  float p;        // drop probability
  float scale;    // 1 / (1 - p)
  uint64_t seed;  // keep decisions are a function of (seed, b, h, row, entry)
};

// Arguments of the per-row gather forward.
struct GatherArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int64_t qsb, qsh, qss;
  int64_t ksb, ksh, kss;
  int64_t vsb, vsh, vss;
  int64_t osb, osh, oss;
  int64_t lsb, lsh;
  int B, H, groups, q_len, kv_len, D;
  float sm_scale;
  int elem;  // Elem of q, k, v, o (0 float32, 1 bfloat16, 2 float16)
  IndexSource src;
  DropoutArgs drop;
  // naive-path attention weights [B, H, q_len, w] in q's type (may be NULL;
  // written by launch_gather_weights from the forward's lse)
  void* weights;
  int64_t wsb, wsh, wss;
};

// Arguments of the gather backward (any index source, float32 / bfloat16 /
// float16): per-row pass (dQ and each entry's dK / dV coefficients), a stable
// sort of the (kv head, key) of every valid entry, then a key-major pass.
struct GatherBwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  const float* lse;
  int64_t qsb, qsh, qss;
  int64_t ksb, ksh, kss;
  int64_t vsb, vsh, vss;
  int64_t osb, osh, oss;
  int64_t dosb, dosh, doss;
  int64_t dqsb, dqsh, dqss;
  int64_t dksb, dksh, dkss;
  int64_t dvsb, dvsh, dvss;
  int64_t lsb, lsh;
  int B, H, Hkv, groups, q_len, kv_len, D;
  float sm_scale;
  int elem;
  IndexSource src;
  DropoutArgs drop;
  int64_t E;          // entries per batch element: H * q_len * w
  float* cp;          // [B][E] dV coefficient of each entry (dropout-scaled p)
  float* cs;          // [B][E] dK coefficient of each entry (sm_scale * dS)
  uint32_t* keys_in;  // [E] kv_head * kv_len + key of a valid in-range entry, else the sentinel
  uint32_t* vals_in;  // [E] entry ids 0 .. E - 1
  uint32_t* keys_out;
  uint32_t* vals_out;
  int32_t* seg;       // [Hkv * kv_len + 1] start of each (kv head, key) in the sorted order
  int32_t* hist;      // radix sort: digit counts per tile, then their scan (offs)
  int32_t* offs;
  int32_t* parts;     // chunk sums of the scan
  int key_bits;       // bits of the sort keys
};

// Arguments of the block-sparse MFMA backward (bf16).
struct BwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;     // forward output (q's layout strides below)
  const uint16_t* dout;  // gradient of o
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  const float* lse;      // forward log-sum-exp, natural log, [B, H, q_len]
  float* delta;          // workspace [B, H, qpad]: rowsum(dO * O) (then lse2)
  const uint32_t* mask_t;  // [tiles][4 query sub-blocks][128 keys] key-major tile masks
  const uint32_t* qmask;   // [tiles][128 rows][4 words] row-major tile masks, or NULL (walk)
  int64_t qsb, qsh, qss;
  int64_t ksb, ksh, kss;
  int64_t vsb, vsh, vss;
  int64_t osb, osh, oss;
  int64_t dosb, dosh, doss;
  int64_t dqsb, dqsh, dqss;
  int64_t dksb, dksh, dkss;
  int64_t dvsb, dvsh, dvss;
  int64_t lsb, lsh;
  int B, H, Hkv, groups, q_len, kv_len;
  int qpad;  // row stride of delta and lse2 per (b, h): q_len rounded up to 32, + 32
  int nqb, nq, nkb;
  float sm_scale, scale_log2;
  PatternConsts pc;
  const int32_t* row_ptr;   // forward layout (CSR of key tiles per (h, qb))
  const int32_t* col_idx;
  const int32_t* q_items;   // dQ work list (esa_plan_schedule)
  const int32_t* tile_row;  // per layout tile t: h * nqb + qb
  const int32_t* kv_ptr;    // [Hkv * nkb + 1]: tiles of each (kv head, key block)
  const int32_t* kv_tiles;  // layout tile ids, grouped by (kv head, key block)
  const int32_t* kv_items;  // dK/dV work list: (b * Hkv + kvh) * nkb + kb, -1 = idle
  // band-gathered dQ (when q_items is NULL): 16-row groups per (b, h), all
  // groups, groups per XCD range
  int ng, n_groups, per_xcd;
  // band-gathered dK / dV (when kv_items is NULL): 16-key blocks per
  // (b, kv head), all blocks, consecutive blocks per XCD chunk
  int nkb16, n_kblk, kchunk;
  // key blocks 0 .. split_blocks - 1 of each (b, kv head) split over
  // split_parts waves (1: not split); n_bkv = B * Hkv; n_extra workgroups (a
  // multiple of 8) run the parts after the first; part_buf: float32 partial
  // sums [n_bkv][split_blocks][split_parts][2][D / 16][4][64]; part_cnt:
  // arrivals [n_bkv][split_blocks]
  int split_parts, split_blocks, n_bkv, n_extra;
  float* part_buf;
  int* part_cnt;
  int elem;  // Elem of the 16-bit tensors: bf16 or f16
  // non-finite output flags (workspace): one byte per 16-row dQ group
  // ((b * H + h) * ng + row / 16) then one per 16-key dK / dV block (n_qflags
  // + (b * Hkv + kvh) * nkb16 + key / 16), each written 0 or 1 by the kernel
  // that stores the unit; bwd_fix_kernel recomputes the flagged units
  uint8_t* flags;
  int n_qflags, n_kvflags;
  // entry rotation of the band dQ / dK-dV walks, in 64ths of an entry per
  // group or block dispatched on an XCD (set by their launchers)
  int rot_dq, rot_dkdv;
};

// Entry rotation rate of a band kernel's launch (64ths of an entry per unit
// dispatched on an XCD).  A grid of many rounds of resident waves refills
// them one unit at a time, and `rate`, a little ahead of 64 / (resident
// waves per XCD), keeps the resident units on neighbouring entries, whose
// rows share L2.  A grid of up to four rounds starts each round nearly at
// once, where the same rate spreads a round over all 64 entries: when a
// head's gathered rows exceed an XCD's 4 MB L2 such a grid (up to
// max_rounds) takes `few` instead (0, or a small rate that the waves' drift
// over a few rounds favours).
inline int band_rotation(int64_t units, int64_t resident_per_xcd, int64_t head_bytes, int rate,
                         int few, int max_rounds = 4) {
  return units <= max_rounds * 8 * resident_per_xcd && head_bytes > (int64_t(4) << 20) ? few
                                                                                     : rate;
}

hipError_t launch_indices(const PatternConsts& pc, int row0, int nrows, void* indices, void* mask,
                          int elem_bytes, hipStream_t stream);
hipError_t launch_dense_mask(const PatternConsts& pc, int row0, int nrows, int ncols,
                             uint8_t* mask, int64_t stride_h, int64_t stride_s,
                             hipStream_t stream);
hipError_t launch_layout(const PatternConsts& pc, const LayoutDims& ld, int32_t* row_ptr,
                         int32_t* col_idx, void* workspace, hipStream_t stream);
// per-stage row masks of a 64 x 32 or 128 x 64 layout: num_tiles x block_m x
// (block_n / 32) words
hipError_t launch_stage_masks(const PatternConsts& pc, const LayoutDims& ld, const int32_t* row_ptr,
                              const int32_t* col_idx, uint32_t* masks, hipStream_t stream);
hipError_t launch_tile_fwd(const TileArgs& a, int head_dim, int64_t num_items,
                           hipStream_t stream);
hipError_t launch_band_fwd(const BandArgs& a, int head_dim, hipStream_t stream);
// the sliding-window kernel takes the band forward's layer-0 prefills
bool window_fwd_applies(const BandArgs& a, int head_dim);
hipError_t launch_window_fwd(const BandArgs& a, int head_dim, hipStream_t stream);
// prep: the kernel forms and stores delta / lse2 itself (see band_dq_kernel)
hipError_t launch_bwd_fix(const BwdArgs& a, int head_dim, hipStream_t stream);
hipError_t launch_band_dq(const BwdArgs& a, int head_dim, const float* lse2, bool prep,
                          hipStream_t stream);
hipError_t launch_band_dkdv(const BwdArgs& a, int head_dim, const float* lse2,
                            hipStream_t stream);
hipError_t launch_gather_fwd(const GatherArgs& a, bool pattern, hipStream_t stream);
hipError_t launch_gather_weights(const GatherArgs& a, bool pattern, hipStream_t stream);
// int32 entries of the sort's digit histograms (and of their scan) and of
// its scan's chunk sums, for n pairs
void gather_bwd_sort_sizes(int64_t n, int64_t* hist_ints, int64_t* part_ints);
hipError_t launch_gather_bwd(const GatherBwdArgs& a, bool pattern, hipStream_t stream);
hipError_t launch_tile_masks(const PatternConsts& pc, const int32_t* row_ptr, const int32_t* col_idx,
                             int nqb, int q_len, uint32_t* mask_t, hipStream_t stream);
hipError_t launch_reachability(const PatternConsts* layers, int num_layers, int position,
                               uint32_t* reach, uint32_t* work, int32_t* counts,
                               hipStream_t stream);
hipError_t launch_tile_bwd(const BwdArgs& a, int head_dim, int64_t num_q_items,
                           int64_t num_kv_items, hipStream_t stream);

}  // namespace esa
