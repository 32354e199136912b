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
  float scale_log2;  // sm_scale * log2(e)
  PatternConsts pc;
  const int32_t* row_ptr;
  const int32_t* col_idx;
  const int32_t* items;
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
  int w;  // entries per row
  // pattern source
  PatternConsts pc;
  const int64_t* positions;  // may be NULL (row r is position r)
  // explicit-index source
  const void* indices;
  const void* mask;
  int index_bytes, mask_bytes;
  int64_t ish, iss, msh, mss;
};

hipError_t launch_indices(const PatternConsts& pc, int row0, int nrows, void* indices, void* mask,
                          int elem_bytes, hipStream_t stream);
hipError_t launch_layout(const PatternConsts& pc, const LayoutDims& ld, int32_t* row_ptr,
                         int32_t* col_idx, void* workspace, hipStream_t stream);
hipError_t launch_tile_fwd(const TileArgs& a, int head_dim, int64_t num_items,
                           hipStream_t stream);
hipError_t launch_gather_fwd(const GatherArgs& a, bool f32, bool pattern, hipStream_t stream);

}  // namespace esa
