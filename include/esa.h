/*
 * Elastic sparse attention forward for AMD MI355X (gfx950) -- C ABI.
 *
 * Library: libesa.so (built from elastic-sparse-attention_amd/csrc).
 *
 * Conventions shared by every entry point:
 *   - Every function returns an esa_status; 0 (ESA_OK) means success.  Invalid
 *     arguments are rejected on the host before anything is launched.
 *   - Device pointers are plain addresses of device memory the caller owns.
 *     The library never allocates device memory.  Its one piece of mutable
 *     global state is the per-device workspace array of
 *     esa_elastic_bwd_noalloc: calls of that entry point that overlap in
 *     time on one device race on it.  Every other call may run concurrently
 *     with any other on different streams.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Launch functions are asynchronous and never synchronise the host.
 *   - Strides are in elements.  The innermost (head_dim / w) dimension of
 *     every tensor is contiguous.
 *
 * Each entry point names the part of the reference's
 * elastic_sparse_attention.py (HighCWu/elastic-sparse-attention) it replaces.
 */
#ifndef ESA_H_
#define ESA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t esa_status;
#define ESA_OK 0
#define ESA_ERR_NULL 1        /* a required pointer is NULL */
#define ESA_ERR_SHAPE 2       /* inconsistent or out-of-range sizes */
#define ESA_ERR_DTYPE 3       /* unsupported element type */
#define ESA_ERR_ALIGN 4       /* pointer or stride misaligned for the kernel */
#define ESA_ERR_UNSUPPORTED 5 /* valid request this build has no kernel for */
#define ESA_ERR_CAPACITY 6    /* output or workspace buffer too small */
#define ESA_ERR_HIP 7         /* a HIP runtime call failed */

typedef int32_t esa_dtype;
#define ESA_F32 0
#define ESA_BF16 1
#define ESA_F16 2

/* Elastic pattern parameters: the constructor arguments that fix the index
 * set (elastic_sparse_attention.py:375-386, used at :477-535) plus the tile
 * shape of the block layout. */
typedef struct esa_pattern {
  int32_t seq_len;           /* rows (query positions 0..seq_len-1) covered */
  int32_t attention_length;  /* w: keys per query row */
  int32_t layer_idx;         /* 0-based layer index */
  int32_t num_hidden_layers; /* layers in the model */
  int32_t num_heads;         /* query heads H */
  int32_t block_m;           /* query rows per tile (layout granularity) */
  int32_t block_n;           /* keys per tile (layout granularity) */
} esa_pattern;

/* q, k, v, o and the log-sum-exp of one forward call.  Mirrors the tensors
 * ElasticSparseAttentionFunction.forward receives and allocates
 * (elastic_sparse_attention.py:241-257): q [B, H, Lq, D], k and v
 * [B, Hkv, Lk, D]; o has q's shape and dtype but any (b, h, s) strides, so
 * [B, Lq, H, D] can be written directly; lse is float32 [B, H, Lq] with
 * contiguous s (may be NULL). */
typedef struct esa_fwd_args {
  esa_dtype dtype; /* element type of q, k, v and o */
  int32_t batch, num_heads, num_kv_heads, q_len, kv_len, head_dim;
  const void* q;
  int64_t q_stride_b, q_stride_h, q_stride_s;
  const void* k;
  int64_t k_stride_b, k_stride_h, k_stride_s;
  const void* v;
  int64_t v_stride_b, v_stride_h, v_stride_s;
  void* o;
  int64_t o_stride_b, o_stride_h, o_stride_s;
  float* lse;
  int64_t lse_stride_b, lse_stride_h;
  float sm_scale; /* the module's scaling = head_dim ** -0.5 (:444) */
} esa_fwd_args;

/* Host only.  Set-up of the library on one device (an index below
 * hipGetDeviceCount): looks up, with that device current, the device address
 * of the array esa_elastic_bwd_noalloc uses as its workspace
 * (hipGetSymbolAddress, which also loads the library's code object there),
 * and keeps it; the caller's current device is restored.  Allocates nothing.
 * Call it once per device before capturing esa_elastic_bwd_noalloc into a
 * HIP graph: without it, the entry point's first call on a device does the
 * lookup, which must not happen under capture.  Calling it again is
 * harmless.  No reference counterpart. */
esa_status esa_init_device(int32_t device);

/* Human-readable name of a status code. */
const char* esa_status_string(esa_status s);

/* Library version string. */
const char* esa_version(void);

/* Host only.  Checks an esa_pattern and reports the sizes of its block
 * layout: query blocks per head, key blocks, an upper bound on the number of
 * active tiles (the col_idx capacity esa_build_layout needs) and the
 * workspace esa_build_layout needs.  A pattern whose bound exceeds INT32_MAX
 * is rejected (ESA_ERR_SHAPE): tile ids and row_ptr are int32.  No reference
 * counterpart: the reference never forms a block layout. */
esa_status esa_layout_sizes(const esa_pattern* p, int32_t* num_qblocks,
                            int32_t* num_kblocks, int64_t* max_tiles,
                            size_t* workspace_bytes);

/* Replaces ElasticSparseAttention._create_elastic_sparse_indices
 * (elastic_sparse_attention.py:470-535).  Writes rows [row0, row0 + nrows)
 * of the index set as indices[H, nrows, w] (masked entries 0, :533) and
 * mask[H, nrows, w] (1 = valid), each with elem_bytes = 4 (int32) or 8
 * (int64, the reference's dtype).  Either output may be NULL.  Bit-exact with
 * the reference's torch float32 evaluation. */
esa_status esa_build_indices(const esa_pattern* p, int32_t row0, int32_t nrows,
                             void* indices, void* mask, int32_t elem_bytes,
                             void* stream);

/* Replaces ElasticSparseAttention._create_full_sparse_mask
 * (elastic_sparse_attention.py:537-572), the dense boolean mask the
 * reference's "dense" implementation hands to SDPA: for rows
 * [row0, row0 + nrows) of the index set and every head h, writes the bytes
 * mask[h * stride_h + r * stride_s + c], c in [0, ncols): 1 where row
 * row0 + r has a valid entry with index c (indices clamped to
 * [0, ncols - 1], :556), else 0.  Every byte of each row's ncols is
 * written, none between rows.  stride_s >= ncols, stride_h >= nrows *
 * stride_s (for more than one head).  Bit-exact with the reference's mask,
 * which is built from the same index set. */
esa_status esa_build_dense_mask(const esa_pattern* p, int32_t row0, int32_t nrows,
                                int32_t ncols, uint8_t* mask, int64_t stride_h,
                                int64_t stride_s, void* stream);

/* Block layout builder (derived from :470-535; no reference counterpart).
 * For every (head h, query block qb) writes the ascending list of active key
 * tiles -- tiles kb with some valid index idx of a row in the block and
 * idx / block_n == kb -- as CSR: row_ptr[H * nqb + 1] (rows ordered
 * h * nqb + qb) and col_idx[row_ptr[H * nqb]].  col_capacity is the length
 * of col_idx; the workspace is at least esa_layout_sizes' figure. */
esa_status esa_build_layout(const esa_pattern* p, int32_t* row_ptr,
                            int32_t* col_idx, int64_t col_capacity,
                            void* workspace, size_t workspace_bytes,
                            void* stream);

/* Host only.  Work list for esa_elastic_fwd: the (batch, head, query block)
 * items of a forward over q_len query rows, laid out for the device.
 * Replaces the implicit Triton grid (q_len, H, B)
 * (elastic_sparse_attention.py:261).  row_ptr_host is esa_build_layout's
 * row_ptr copied to host memory.  Item b * H * nqb + h * nqb + qb appears
 * exactly once; the list is cut into 8 runs of equal tile count, one per
 * XCD (workgroup id % 8), each run walking whole (batch, head) streams with
 * their query blocks longest first, and shorter runs padded with -1 (an
 * idle workgroup).  With items_host NULL only *num_items (the list length,
 * at most 8 * batch * H * ceil(q_len / block_m)) is written. */
esa_status esa_plan_schedule(const esa_pattern* p, const int32_t* row_ptr_host,
                             int32_t q_len, int32_t batch, int32_t* items_host,
                             int64_t items_capacity, int64_t* num_items);

/* Block-sparse forward over the elastic pattern, query rows at positions
 * 0..q_len-1.  Replaces _triton_forward + ElasticSparseAttentionFunction
 * .forward (elastic_sparse_attention.py:592-622, 241-297) for prefill.
 * Visits only the active key blocks of the layout, runs QK^T and PV on bf16
 * MFMA with float32 accumulation and online softmax.  The layout's block
 * shape is the staging unit: 128 x 128 (whole tiles), 128 x 64 (four waves
 * per 128 query rows, 64-key stages) or 64 x 32 (two waves per 64 query
 * rows, 32-key stages, the fastest in general); in the finer layouts the
 * parts of a 128-key tile that no row of the query block needs are never
 * staged.  All give the same output bit for bit.  Requires dtype ESA_BF16
 * or ESA_F16 (the MFMAs and P in that type, float32 accumulation),
 * head_dim 64 or 128, (block_m, block_n) in {(128, 128), (128, 64),
 * (64, 32)}, a finite sm_scale > 0
 * (ESA_ERR_UNSUPPORTED otherwise; esa_elastic_fwd_rows takes any), K and V
 * row strides >= head_dim with kv_len * row stride * 2 < 2^31 (one head's
 * rows within a 2 GiB window), q_len <= kv_len,
 * q_len <= p->seq_len, 16-byte aligned rows.  items/num_items come from
 * esa_plan_schedule (copied to device memory); item ids outside the forward
 * are skipped.  stage_masks: NULL (each row's valid keys per stage are
 * computed in the kernel from the pattern), or, for a 64 x 32 or 128 x 64
 * layout, the masks esa_build_stage_masks wrote for this layout (8-byte
 * aligned); same output bit for bit, without the per-row index walk.  With
 * stage_masks, stage_mask_words is their length in 32-bit words and
 * row_ptr_host the host copy of row_ptr: a buffer shorter than
 * esa_stage_masks_size(p, row_ptr_host) is rejected (ESA_ERR_CAPACITY), a
 * NULL row_ptr_host too (ESA_ERR_NULL); without stage_masks both are
 * ignored. */
esa_status esa_elastic_fwd(const esa_fwd_args* a, const esa_pattern* p,
                           const int32_t* row_ptr, const int32_t* col_idx,
                           const int32_t* row_ptr_host,
                           const uint32_t* stage_masks, int64_t stage_mask_words,
                           const int32_t* items, int64_t num_items, void* stream);

/* Host only.  32-bit words of the stage masks of a 64 x 32, 128 x 64 or
 * 128 x 128 layout (block_m x block_n of p): num_tiles x block_m x
 * block_n / 32, with num_tiles = row_ptr_host[num_heads * num_qblocks]. */
esa_status esa_stage_masks_size(const esa_pattern* p, const int32_t* row_ptr_host,
                                int64_t* words);

/* Per-stage row masks of a 64 x 32 or 128 x 64 layout, for esa_elastic_fwd,
 * or of a 128 x 128 layout, for esa_elastic_bwd's block-sparse dQ: for stage
 * (key block) st of the layout and query row r of its block, the
 * row's valid keys among the block's keys as block_n / 32 words at
 * masks[(st * block_m + r) * block_n / 32 ..].  The bits of
 * _create_elastic_sparse_indices (elastic_sparse_attention.py:470-535), as
 * the forward's in-kernel walk computes them, once per layout instead of
 * once per batch element and forward.  row_ptr / col_idx from
 * esa_build_layout with the same pattern, row_ptr_host its host copy;
 * capacity_words >= esa_stage_masks_size. */
esa_status esa_build_stage_masks(const esa_pattern* p, const int32_t* row_ptr,
                                 const int32_t* col_idx, const int32_t* row_ptr_host,
                                 uint32_t* masks, int64_t capacity_words, void* stream);

/* Band-gathered forward over the elastic pattern, prefill rows 0 .. q_len-1,
 * or the rows at positions[r] (int64 device array, as cache_position,
 * :602-608; NULL = rows 0 .. q_len-1) (no layout needed).  Replaces the
 * forward branch of the Triton kernel (elastic_sparse_attention.py:117-166)
 * as _triton_forward launches it for prefill and chunked prefill (:592-622),
 * with each row's index list regenerated on the device (bit-exact with
 * :470-535).  With positions, each group of 16 rows whose positions are
 * consecutive and in [0, kv_len) (negative ones counting from kv_len) runs
 * as below from its first row's position; any other group computes its rows
 * one at a time with esa_elastic_fwd_rows' arithmetic (float32), a row whose
 * position lies outside [-kv_len, kv_len) getting NaN; q_len and kv_len are
 * then not compared.  Entry j of the rows' index lists (a band)
 * moves by at most one key per row (two at a few rows of some heads), so 16
 * consecutive rows mostly use at most 16 consecutive keys of each band
 * (wider bands are handled, more slowly):
 * one wave gathers each band's keys once for its 16 rows and runs QK^T and
 * PV on bf16 MFMA with float32 accumulation and online softmax.  At
 * interpolation weight 0 (layer 0: every row attends the keys
 * max(0, i - w + 1) .. i) with head_dim 64 or 128, a sliding-window kernel
 * runs instead: one wave per 32 rows (groups of 32 at positions), each key
 * of their windows staged once.  Same outputs as esa_elastic_fwd within
 * bf16 rounding.  Requires dtype
 * ESA_BF16 or ESA_F16, head_dim a multiple of 8 up to 256 (kernels at 64,
 * 128 and 256; other head dims run the next of them with zero padding),
 * attention_length <= 64, kv_len < 2^24,
 * (kv_len + 16) * K/V row stride * 2 < 2^31, row strides >= head_dim,
 * q_len <= kv_len, q_len <= p->seq_len, finite sm_scale > 0, 16-byte
 * aligned q, k, v, o and strides (elements) that are multiples of 8. */
esa_status esa_elastic_fwd_band(const esa_fwd_args* a, const esa_pattern* p,
                                const int64_t* positions, void* stream);

/* Per-row gather forward over the elastic pattern for arbitrary query
 * positions: row r of q is position positions[r] (int64 device array, as
 * cache_position, :602-608), or r when positions is NULL.  Replaces the
 * decode branch of _triton_forward (:602-619).  Each row's w indices are
 * regenerated on the device (bit-exact with :470-535) and clamped to
 * [0, kv_len - 1] (:615).  Positions index rows [0, kv_len) of the index set
 * (:588, :602-608), a negative position counting from kv_len as torch
 * indexing counts it; a row whose position lies outside [-kv_len, kv_len)
 * (the reference's indexing error) gets NaN output and NaN lse, so the call
 * never synchronises to check positions.  dtype ESA_F32, ESA_BF16 or ESA_F16
 * (computed in float32, stored in the inputs' type, as the Triton kernel
 * does, :114, :163), head_dim a multiple of 4, <= 256. */
esa_status esa_elastic_fwd_rows(const esa_fwd_args* a, const esa_pattern* p,
                                const int64_t* positions, void* stream);

/* Options of the naive path's forward (implementation="naive",
 * elastic_sparse_attention.py:624-680). */
typedef struct esa_naive_opts {
  float dropout_p; /* attention dropout in [0, 1) (:674); 0 = none */
  uint64_t seed;   /* keep decisions are a function of (seed, b, h, row, entry) */
  void* weights;   /* [B, H, q_len, w] in the inputs' type, or NULL */
  int64_t weights_stride_b, weights_stride_h, weights_stride_s;
} esa_naive_opts;

/* Replaces _naive_forward (:624-680): esa_elastic_fwd_rows plus the
 * attention weights it returns, softmax(scores) over each row's entries
 * (masked entries 0, :669-673), and attention dropout on them (:674): each
 * probability is kept with probability 1 - dropout_p and then scaled by
 * 1 / (1 - dropout_p), and O is formed from the kept weights.  lse is that
 * of the undropped probabilities.  With opts->weights non-NULL, a->lse must
 * be non-NULL (the weights are exp(s - lse)).  The keep decisions are a
 * counter-based hash of (seed, b, h, row, entry), so esa_elastic_bwd_rows
 * with the same seed reproduces them; they are not torch's random stream. */
esa_status esa_elastic_fwd_naive(const esa_fwd_args* a, const esa_pattern* p,
                                 const int64_t* positions, const esa_naive_opts* opts,
                                 void* stream);

/* Gather forward over explicit index lists: the operator
 * ElasticSparseAttentionFunction.forward(q, k, v, sparse_indices,
 * sparse_mask, sm_scale, num_kv_groups) (elastic_sparse_attention.py:241-297).
 * indices [H, q_len, attn_length] with index_bytes 4 or 8, mask
 * [H, q_len, attn_length] with mask_bytes 1, 4 or 8 (nonzero = valid).
 * Query head h reads kv head h / (H / Hkv) (:89).  Semantics of the Triton
 * kernel (:117-166): a valid entry whose index lies outside [0, kv_len)
 * scores 0 against a zero key and value; an entry listed twice counts twice.
 * A row with no valid entry gets output 0 and lse -inf. */
esa_status esa_sparse_fwd(const esa_fwd_args* a, const void* indices,
                          int32_t index_bytes, int64_t idx_stride_h,
                          int64_t idx_stride_s, const void* mask,
                          int32_t mask_bytes, int64_t mask_stride_h,
                          int64_t mask_stride_s, int32_t attn_length,
                          void* stream);

/* Tensors of one backward call over the elastic pattern: the forward's
 * inputs, its output o (any strides, as esa_elastic_fwd wrote it) and
 * log-sum-exp, the incoming gradient dout (o's shape), and the gradients to
 * write: dq (q's shape), dk and dv (k's shape).  Mirrors what
 * ElasticSparseAttentionFunction.backward receives and returns
 * (elastic_sparse_attention.py:299-339).  All bf16 except lse (float32,
 * natural log, [B, H, q_len] with contiguous rows). */
typedef struct esa_bwd_args {
  esa_dtype dtype; /* ESA_BF16 or ESA_F16 (esa_elastic_bwd); any (gather backward) */
  int32_t batch, num_heads, num_kv_heads, q_len, kv_len, head_dim;
  const void* q;
  int64_t q_stride_b, q_stride_h, q_stride_s;
  const void* k;
  int64_t k_stride_b, k_stride_h, k_stride_s;
  const void* v;
  int64_t v_stride_b, v_stride_h, v_stride_s;
  const void* o;
  int64_t o_stride_b, o_stride_h, o_stride_s;
  const void* dout;
  int64_t dout_stride_b, dout_stride_h, dout_stride_s;
  void* dq;
  int64_t dq_stride_b, dq_stride_h, dq_stride_s;
  void* dk;
  int64_t dk_stride_b, dk_stride_h, dk_stride_s;
  void* dv;
  int64_t dv_stride_b, dv_stride_h, dv_stride_s;
  const float* lse;
  int64_t lse_stride_b, lse_stride_h;
  float sm_scale;
} esa_bwd_args;

/* Host only.  Work lists of the backward (no reference counterpart: the
 * reference scatters dK and dV with atomics from a (q_len, H, B) grid,
 * :299-339).  From esa_build_layout's row_ptr and col_idx (host copies) and
 * q_len, batch and num_kv_heads, writes
 *   tile_row[T]         T = row_ptr[H * nqb]: h * nqb + qb of layout tile t
 *   kv_ptr[Hkv * nkb + 1], kv_tiles[*num_kv_tiles]: for each (kv head,
 *                       key block), the layout tiles of query blocks below
 *                       ceil(q_len / 128) of its query heads that hold the
 *                       key block, in (head, query block) order
 *   kv_items[*num_kv_items]: (b * Hkv + kvh) * nkb + kb work items laid out
 *                       for the 8 XCDs like esa_plan_schedule's, -1 = idle.
 * With any of tile_row, kv_ptr, kv_tiles, kv_items NULL only the two counts
 * are written. */
esa_status esa_plan_bwd(const esa_pattern* p, const int32_t* row_ptr_host,
                        const int32_t* col_idx_host, int32_t q_len,
                        int32_t batch, int32_t num_kv_heads,
                        int32_t* tile_row, int32_t* kv_ptr,
                        int32_t* kv_tiles, int64_t kv_tiles_capacity,
                        int32_t* kv_items, int64_t kv_items_capacity,
                        int64_t* num_kv_tiles, int64_t* num_kv_items);

/* Key-major masks of the active layout tiles a backward over q_len query
 * rows reads: mask_t[t * 512 + qs * 128 + k] bit r is set when query row
 * qb * 128 + 32 qs + r (< q_len) has key col_idx[t] * 128 + k among its
 * valid elastic entries (:470-535), for every tile t of a query block
 * qb < ceil(q_len / 128).  row_ptr_host is the host copy of row_ptr; mask_t
 * must hold row_ptr_host[(H - 1) * nqb + ceil(q_len / 128)] * 512 uint32
 * (mask_capacity), the end of the last head's tiles among those blocks.
 * Depends only on the pattern and q_len, so it can be built once and
 * reused. */
esa_status esa_build_tile_masks(const esa_pattern* p, const int32_t* row_ptr,
                                const int32_t* col_idx, const int32_t* row_ptr_host,
                                int32_t q_len, uint32_t* mask_t,
                                int64_t mask_capacity, void* stream);

/* Host only.  Bytes of workspace esa_elastic_bwd needs:
 * 2 * batch * num_heads * qpad floats, qpad = q_len rounded up to 32, plus
 * 32 (per-row delta and log2 LSE), and, when the band dK/dV may split key
 * block 0 (num_heads / num_kv_heads * q_len > 6144), P float32 partial
 * sums of 2 * 16 * head_dim floats and one counter per (batch, kv head),
 * P = that product / 6144 rounded up, at most 32, then, from the next
 * 256-byte boundary, one byte per 16-row dQ group (batch * num_heads *
 * ceil(q_len / 16)) and per 16-key dK / dV block (batch * num_kv_heads *
 * ceil(kv_len / 16)): the kernels' non-finite flags.  The total is a
 * multiple of 256.  Requires num_kv_heads and head_dim >= 1. */
esa_status esa_bwd_workspace_size(const esa_bwd_args* a, size_t* workspace_bytes);

/* Backward over the elastic pattern: replaces the backward branch of the
 * Triton kernel (elastic_sparse_attention.py:168-233) and
 * ElasticSparseAttentionFunction.backward (:299-339) for the prefill
 * forward (esa_elastic_fwd or esa_elastic_fwd_band: any O and LSE of it).  Writes dq, dk and dv (every element; no
 * zero-initialisation needed, and deterministic: each gradient row is
 * accumulated by one workgroup in a fixed order, except that at the last
 * layer (alpha = 1) the band dK/dV splits key block 0 over several waves
 * whose float32 sums the last to arrive (an atomic counter in the
 * workspace) adds in part order; no atomics on the gradients).
 * q_items/num_q_items: esa_plan_schedule's list for (q_len, batch), for a
 * block-sparse dQ over the layout row_ptr/col_idx; q_items NULL computes dQ
 * with the band-gathered kernel instead (as esa_elastic_fwd_band gathers:
 * attention_length <= 64, kv_len < 2^24; num_q_items is ignored).
 * tile_row, kv_ptr, kv_tiles, kv_items/num_kv_items: esa_plan_bwd's, and
 * mask_t: esa_build_tile_masks' for this q_len, for a block-sparse dK/dV;
 * kv_items NULL computes dK and dV with the band-gathered key-major kernel
 * instead (same limits; tile_row, kv_ptr, kv_tiles, mask_t and num_kv_items
 * are ignored).  With both NULL no layout is read (row_ptr, col_idx may be
 * NULL).  At interpolation weight 0 (layer_idx 0: a sliding window, row i
 * attends keys max(0, i - w + 1) .. i) both band kernels walk the window's
 * key chunks and row ranges directly.  q_masks: NULL (the block-sparse dQ computes each row's valid keys
 * per tile from the pattern), or esa_build_stage_masks' masks of this 128 x
 * 128 layout (16-byte aligned; only with q_items, ESA_ERR_UNSUPPORTED
 * otherwise): same results bit for bit, without the per-row index walk.
 * All lists and masks are device memory.  mask_t_words and q_mask_words are
 * the lengths of mask_t and q_masks in 32-bit words, checked on the host
 * against what the kernels read (mask_t: esa_build_tile_masks' size for
 * q_len; q_masks: esa_stage_masks_size) from row_ptr_host, the host copy of
 * row_ptr, which is required (ESA_ERR_NULL) whenever mask_t or q_masks is
 * read; a shorter buffer is rejected (ESA_ERR_CAPACITY).
 * Inf and NaN in the inputs reach exactly the gradients the reference's
 * gather reaches: each kernel flags the 16-row dQ groups and 16-key dK / dV
 * blocks it stores with a non-finite value, and a last kernel recomputes
 * those on the listed (row, entry) pairs only.
 * Requires dtype ESA_BF16 or ESA_F16, head_dim 64 or 128, block 128 x 128, a finite
 * sm_scale > 0, q_len <= kv_len, 16-byte aligned rows. */
esa_status esa_elastic_bwd(const esa_bwd_args* a, const esa_pattern* p,
                           const int32_t* row_ptr, const int32_t* col_idx,
                           const int32_t* row_ptr_host,
                           const int32_t* q_items, int64_t num_q_items,
                           const int32_t* tile_row, const int32_t* kv_ptr,
                           const int32_t* kv_tiles, const int32_t* kv_items,
                           int64_t num_kv_items, const uint32_t* mask_t,
                           int64_t mask_t_words, const uint32_t* q_masks,
                           int64_t q_mask_words, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Host only.  Bytes of workspace esa_sparse_bwd and esa_elastic_bwd_rows
 * need for index lists of attn_length entries per row: per batch element and
 * entry two float32 coefficients, four uint32 arrays of entries for the sort,
 * (num_kv_heads * kv_len + 1) int32 segment starts, and the sort's
 * histograms (each region 256-byte aligned).  Requires num_heads * q_len *
 * attn_length and num_kv_heads * kv_len below 2^31 - 1. */
esa_status esa_gather_bwd_workspace_size(const esa_bwd_args* a, int32_t attn_length,
                                         size_t* workspace_bytes);

/* Backward of the operator over explicit index lists: replaces
 * ElasticSparseAttentionFunction.backward (elastic_sparse_attention.py:
 * 299-339) and the Triton kernel's backward branch (:168-233) with the same
 * indices / mask arguments as esa_sparse_fwd, o and lse of that forward, and
 * dout.  Writes dq, dk and dv (every element of dk and dv: keys no entry
 * reaches get 0, as the reference's zeros_like does).  Semantics of the
 * reference: p = exp(scale q.k - lse) on valid entries; an entry whose index
 * lies outside [0, kv_len) scores 0 against zero K/V and adds nothing to dk or
 * dv; an entry listed twice counts twice.  No atomics on the gradients: each
 * entry's dK / dV coefficients go to the workspace, a stable radix sort
 * groups them by key, and one wave sums each key's entries in entry order,
 * so results are deterministic.  dtype ESA_F32, ESA_BF16 or ESA_F16
 * (float32 arithmetic), head_dim a multiple of 4 up to 256, K / V rows
 * aligned to 4 elements; workspace from esa_gather_bwd_workspace_size,
 * 256-byte aligned. */
esa_status esa_sparse_bwd(const esa_bwd_args* a, const void* indices, int32_t index_bytes,
                          int64_t idx_stride_h, int64_t idx_stride_s, const void* mask,
                          int32_t mask_bytes, int64_t mask_stride_h, int64_t mask_stride_s,
                          int32_t attn_length, void* workspace, size_t workspace_bytes,
                          void* stream);

/* Backward of esa_elastic_fwd_rows / esa_elastic_fwd_naive (the pattern's
 * rows at positions, or 0 .. q_len-1 when positions is NULL): the gradients
 * of the module's float32, float16, decode and other-head_dim paths and of
 * the naive path with dropout (dropout_p and seed as the forward used them).
 * Same kernels, semantics and workspace as esa_sparse_bwd with the index
 * lists regenerated on the device (masked entries 0, clamped to
 * [0, kv_len - 1], :602-615). */
esa_status esa_elastic_bwd_rows(const esa_bwd_args* a, const esa_pattern* p,
                                const int64_t* positions, float dropout_p, uint64_t seed,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free variant of esa_elastic_bwd, with the same arguments
 * except the workspace.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * training or serving loops, harnesses that forbid hipMalloc).  The
 * workspace is a file-scope device array of esa_bwd_noalloc_max_workspace()
 * bytes (32 MiB) that each device the library runs on holds until the
 * process ends; a call whose esa_bwd_workspace_size exceeds it returns
 * ESA_ERR_CAPACITY before launching anything.  The call allocates nothing
 * and issues no memset: the kernels clear what must start at zero (the split
 * counters).  Every call on one device shares that device's array, so calls
 * that overlap in time on one device (different streams, or host threads)
 * race on it and must be serialised by the caller; consecutive calls on one
 * stream are safe.  Results are bit-identical to esa_elastic_bwd's.  The
 * array's device address is looked up once per device, by esa_init_device
 * or else on the entry point's first call there: a caller that captures its
 * first call into a HIP graph calls esa_init_device before the capture. */
esa_status esa_elastic_bwd_noalloc(const esa_bwd_args* a, const esa_pattern* p,
                                   const int32_t* row_ptr, const int32_t* col_idx,
                                   const int32_t* row_ptr_host,
                                   const int32_t* q_items, int64_t num_q_items,
                                   const int32_t* tile_row, const int32_t* kv_ptr,
                                   const int32_t* kv_tiles, const int32_t* kv_items,
                                   int64_t num_kv_items, const uint32_t* mask_t,
                                   int64_t mask_t_words, const uint32_t* q_masks,
                                   int64_t q_mask_words, void* stream);

/* Bytes of the per-device array esa_elastic_bwd_noalloc uses as its
 * workspace (the largest esa_bwd_workspace_size it accepts).  Host only. */
size_t esa_bwd_noalloc_max_workspace(void);

/* Replaces check_attention_holes_pytorch (check_attn_hole.py:53-180): the
 * tokens `position` reaches through num_hidden_layers elastic layers of
 * num_heads heads (each layer's index set is the pattern of
 * esa_build_indices at that layer_idx).  The last layer starts the set with
 * the position and its valid indices over all heads; every earlier layer, from
 * num_hidden_layers - 2 down to 0, adds the valid indices of every token
 * already in the set.  reach (device, (position + 32) / 32 words) receives bit
 * j % 32 of word j / 32 set iff token j is reachable; work is a device buffer
 * of the same size.  layer_counts (device, num_hidden_layers int32, or NULL)
 * receives the set size after each layer, last layer first.  0 <= position <
 * seq_len (the reference's ValueError).  No index buffers: each pass
 * regenerates the indices.  Asynchronous on `stream`. */
esa_status esa_reachability(int32_t seq_len, int32_t attention_length,
                            int32_t num_hidden_layers, int32_t num_heads,
                            int32_t position, uint32_t* reach, uint32_t* work,
                            int32_t* layer_counts, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ESA_H_ */
