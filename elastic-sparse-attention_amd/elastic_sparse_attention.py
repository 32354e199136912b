"""Elastic sparse attention for AMD MI355X: drop-in for the reference module.

Same class names, constructor arguments, forward signature, return values and
errors as the reference's ``elastic_sparse_attention.py``
(HighCWu/elastic-sparse-attention):

* ``ElasticSparseAttention(layer_idx, num_hidden_layers, num_attention_heads,
  head_dim, attention_length, max_seq_len, num_key_value_heads=None,
  attention_dropout=0.0, implementation="triton")``   (:375-386)
* ``forward(query_states, key_states, value_states, cache_position=None)
  -> (attn_output [B, Lq, H * D], None)``             (:728-765)
* ``ElasticSparseAttentionFunction.apply(q, k, v, sparse_indices,
  sparse_mask, sm_scale, num_kv_groups) -> o [B, H, Lq, D]``  (:241-297)

Underneath, every call goes through libesa.so's C ABI (include/esa.h) to
hand-written gfx950 HIP kernels:

* prefill (``cache_position is None``), bf16 or fp16, head_dim 64 or 128: the
  band-gathered MFMA kernel (each row's index-list entries as 16-key bands;
  at layer 0, a sliding window, its window kernel) or the block-sparse MFMA
  kernel over the block layout (CSR of active 128x128 tiles, built once per
  device by the HIP layout builder), whichever is faster for the shape, or
  the two split by rows (``prefill_split``); other head dims that are
  multiples of 8 up to 256: the band kernel (at D = 256, or padded to 64,
  128 or 256);
* chunked prefill (``cache_position`` of at least 32 rows), bf16 or fp16:
  the band (or window) kernel at those positions, except at a dilated layer
  for calls of at most 3072 · 128 / head_dim (batch, head, row) units, where
  the per-row gather is faster;
* decode (fewer ``cache_position`` rows), float32, or other head dims: the
  per-row gather kernel that regenerates each row's elastic indices on the
  device.

The index cache the reference keeps as two int64 buffers
(``sparse_attention_indices``, ``sparse_causal_mask``, :454-468) is not held
by default: the kernels regenerate indices from the pattern.  The two
attributes are still available and are materialised on first access, on the
GPU, by the HIP index builder.

Differences from the reference, all deliberate:
* ``implementation`` accepts "triton", "naive" and "dense" (anything else is
  the reference's ValueError); all three run the HIP kernels.  "naive"
  returns the attention weights ``[B, H, Lq, w]`` as the reference's naive
  path does (:680; not differentiable here), the others ``None``.  There is
  no CPU path: CPU tensors raise.
* ``attention_dropout`` applies in training mode to "naive" and "dense" (as
  the reference's naive and SDPA paths apply it, :674, :721) and not to
  "triton" (whose kernel ignores it).  Keep decisions come from a
  counter-based hash seeded from torch's generator, not torch's own random
  stream, so the mask differs from torch.dropout's draw for the same seed.
* Every path backpropagates, deterministically (no atomics on the
  gradients): bf16 or fp16 prefill with head_dim 64 or 128 through
  hand-written MFMA kernels (band-gathered, their window forms at layer 0,
  or block-sparse, each half picked per shape); the others (decode and chunked-prefill rows, float32, other
  head dims, dropout, explicit index lists) through the gather backward (row
  pass, stable key sort, key-major pass).
* A query row with no valid entry (impossible for the elastic pattern, only
  reachable through explicit masks) gives output 0 rather than NaN.
* A cache_position on the device is not range-checked on the host (that
  would synchronise); an out-of-range position gives a NaN row.
"""
from __future__ import annotations

import ctypes
import logging
from collections import OrderedDict
from typing import Dict, Optional, Tuple

import torch
import torch.nn as nn

from esa_native import (ESA_BF16, ESA_F16, ESA_F32, EsaBwdArgs, EsaFwdArgs, EsaNaiveOpts,
                        EsaPattern, check, load)

logger = logging.getLogger(__name__)

BLOCK_M = 128
BLOCK_N = 128
# Largest per-stage row masks (bytes) a stage layout keeps for the tile
# forward: 4 bytes per (stage, row), about 8 MB at B=8 H=16 L=4096 layer 4,
# 63 MB at H=32 L=8192 layer 3; longer sequences (where the band kernel runs)
# fall back to the in-kernel walk.
STAGE_MASK_BUDGET = 256 << 20

__all__ = [
    "ElasticSparseAttention",
    "ElasticSparseAttentionFunction",
    "ElasticLayout",
    "make_pattern",
    "build_indices",
    "elastic_attention_fwd",
    "elastic_attention_rows",
    "sparse_attention_fwd",
    "elastic_attention_bwd",
    "init_device",
]


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
# torch's current-stream handle as an integer, without building a Stream
# object (about 2 us per call less on the decode path); the public API where
# this torch build lacks it
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> ctypes.c_void_p:
    if _RAW_STREAM is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return ctypes.c_void_p(_RAW_STREAM(index))
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


_INITIALISED = set()


def init_device(device: torch.device) -> None:
    """esa_init_device on ``device``, once per process: looks up the device
    address of the allocation-free backward's workspace array there (and
    loads the library's kernels), so a later first call of
    ``elastic_attention_bwd(noalloc=True)`` may be captured into a HIP
    graph."""
    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index in _INITIALISED:
        return
    check(load().esa_init_device(index), "esa_init_device")
    _INITIALISED.add(index)


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return ESA_BF16
    if dt == torch.float32:
        return ESA_F32
    if dt == torch.float16:
        return ESA_F16
    raise ValueError(f"unsupported dtype {dt}: the HIP kernels take bfloat16, float16 or "
                     "float32")


def _require_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError(
                "elastic sparse attention runs on the GPU through libesa.so (HIP); "
                f"got a tensor on {t.device}")


def _prep(t: torch.Tensor, align_elems: int) -> torch.Tensor:
    """Innermost dim contiguous, base and strides aligned for row loads."""
    es = t.element_size()
    ok = (t.stride(-1) == 1 and t.data_ptr() % (align_elems * es) == 0
          and all(s % align_elems == 0 for s in t.stride()[:-1]))
    if ok:
        return t
    t = t.contiguous()
    if t.data_ptr() % (align_elems * es) != 0:
        t = t.clone()
    return t


def make_pattern(seq_len: int, attention_length: int, layer_idx: int, num_hidden_layers: int,
                 num_heads: int, block_m: int = BLOCK_M, block_n: int = BLOCK_N) -> EsaPattern:
    """The pattern parameters the C ABI takes (esa_pattern)."""
    return EsaPattern(int(seq_len), int(attention_length), int(layer_idx),
                      int(num_hidden_layers), int(num_heads), int(block_m), int(block_n))


def build_indices(pattern: EsaPattern, device: torch.device, dtype: torch.dtype = torch.int64,
                  row0: int = 0, nrows: Optional[int] = None
                  ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Index set and mask ``[H, nrows, w]`` on ``device``, as
    ``_create_elastic_sparse_indices`` (:470-535) returns them (bit-exact)."""
    lib = load()
    device = torch.device(device)
    _require_gpu(torch.empty(0, device=device))
    nrows = pattern.seq_len - row0 if nrows is None else nrows
    if dtype not in (torch.int64, torch.int32):
        raise ValueError("index dtype must be int64 or int32")
    shape = (pattern.num_heads, nrows, pattern.attention_length)
    idx = torch.empty(shape, dtype=dtype, device=device)
    msk = torch.empty(shape, dtype=dtype, device=device)
    check(lib.esa_build_indices(ctypes.byref(pattern), row0, nrows, ctypes.c_void_p(idx.data_ptr()),
                                ctypes.c_void_p(msk.data_ptr()), idx.element_size(),
                                _stream(device)), "esa_build_indices")
    return idx, msk


class _LRU(OrderedDict):
    """A dict that keeps its ``capacity`` most recently used entries: the
    per-shape caches of a layout stay bounded when a training run feeds many
    distinct sequence lengths or batch sizes."""

    def __init__(self, capacity: int):
        super().__init__()
        self.capacity = int(capacity)

    def get(self, key, default=None):
        if key in self:
            self.move_to_end(key)
            return self[key]
        return default

    def __setitem__(self, key, value):
        super().__setitem__(key, value)
        self.move_to_end(key)
        while len(self) > self.capacity:
            self.popitem(last=False)


class ElasticLayout:
    """Block layout of one elastic pattern on one device.

    ``row_ptr`` (int32 ``[H * nqb + 1]``) and ``col_idx`` (int32) list, for
    every (head, 128-row query block), the ascending 128-key tiles holding at
    least one valid entry.  Built by the HIP layout builder; the host keeps a
    copy of ``row_ptr`` for the work lists (``schedule``, XCD-ordered), one
    per (q_len, batch), cached.
    """

    def __init__(self, pattern: EsaPattern, device: torch.device):
        lib = load()
        self.pattern = pattern
        self.device = torch.device(device)
        nqb = ctypes.c_int32()
        nkb = ctypes.c_int32()
        max_tiles = ctypes.c_int64()
        ws = ctypes.c_size_t()
        check(lib.esa_layout_sizes(ctypes.byref(pattern), ctypes.byref(nqb), ctypes.byref(nkb),
                                   ctypes.byref(max_tiles), ctypes.byref(ws)), "esa_layout_sizes")
        self.num_qblocks = nqb.value
        self.num_kblocks = nkb.value
        H = pattern.num_heads
        self.row_ptr = torch.empty(H * self.num_qblocks + 1, dtype=torch.int32, device=self.device)
        self.col_idx = torch.empty(max(1, max_tiles.value), dtype=torch.int32, device=self.device)
        work = torch.empty(ws.value, dtype=torch.uint8, device=self.device)
        check(lib.esa_build_layout(ctypes.byref(pattern), ctypes.c_void_p(self.row_ptr.data_ptr()),
                                   ctypes.c_void_p(self.col_idx.data_ptr()),
                                   self.col_idx.numel(), ctypes.c_void_p(work.data_ptr()),
                                   ws.value, _stream(self.device)), "esa_build_layout")
        self.row_ptr_host = self.row_ptr.cpu()  # one synchronisation per layout
        del work
        self.num_tiles = int(self.row_ptr_host[-1])
        # col_idx was sized by the bound; keep only the tiles the layout holds
        if self.col_idx.numel() > max(1, self.num_tiles):
            self.col_idx = self.col_idx[:max(1, self.num_tiles)].clone()
        # per-shape caches, each keeping its most recently used entries
        self._schedules = _LRU(self.SCHEDULE_CACHE)   # (q_len, batch) -> work list
        self._col_idx_host: Optional[torch.Tensor] = None
        self._bwd_plans = _LRU(self.PLAN_CACHE)       # (q_len, batch, kv heads) -> plan
        self._masks = _LRU(self.MASK_CACHE)           # q_len -> key-major tile masks
        self._stages = _LRU(self.STAGE_CACHE)         # (block_m, block_n) -> layout
        self._stage_masks = None  # tensor, False (none: over budget), or unbuilt
        self._tiles_for = _LRU(self.COUNT_CACHE)      # q_len -> active tiles
        self._splits = _LRU(self.COUNT_CACHE)         # (q_len, batch, D) -> split row
        self._positions = _LRU(self.SCHEDULE_CACHE)   # (row0, q_len) -> device positions
        self._block_cum = None  # cumulative listed blocks per query block, all heads

    # cache capacities: work lists and backward plans are device arrays sized
    # by the batch and the tile count (about 563K tiles at H=32 L=32768 layer
    # 4), tile masks 2 KB per tile; tile counts are integers
    SCHEDULE_CACHE = 8
    PLAN_CACHE = 4
    MASK_CACHE = 2
    STAGE_CACHE = 3
    COUNT_CACHE = 256

    def stages(self, block_n: int = 32, block_m: Optional[int] = 64) -> "ElasticLayout":
        """The same pattern's layout at ``block_m`` x ``block_n`` blocks, the
        forward's staging unit (64 x 32 by default, or 128 x 64): a part of a
        128 x 128 tile that no row of the query block needs is not listed, so
        the forward never loads it.  Built once per shape, cached; the
        128 x 128 layout itself stays the declared tile (counted flops, the
        backward)."""
        block_m = self.pattern.block_m if block_m is None else block_m
        if self.pattern.block_n == block_n and self.pattern.block_m == block_m:
            return self
        got = self._stages.get((block_m, block_n))
        if got is None:
            p = self.pattern
            got = ElasticLayout(
                make_pattern(p.seq_len, p.attention_length, p.layer_idx, p.num_hidden_layers,
                             p.num_heads, block_m, block_n), self.device)
            self._stages[(block_m, block_n)] = got
        return got

    def stage_masks(self) -> Optional[torch.Tensor]:
        """This layout's per-stage row masks (esa_build_stage_masks), built
        once and cached, for the tile forward (64 x 32 or 128 x 64 stages) or
        the tile backward's dQ (128 x 128 tiles) to load instead of walking
        each row's index list per stage; None for other block shapes or when
        they would exceed STAGE_MASK_BUDGET bytes (then the kernel walks)."""
        if self._stage_masks is False:
            return None
        if self._stage_masks is not None:
            return self._stage_masks
        p = self.pattern
        if (p.block_m, p.block_n) not in ((64, 32), (128, 64), (128, 128)):
            self._stage_masks = False
            return None
        lib = load()
        words = ctypes.c_int64()
        rp = ctypes.c_void_p(self.row_ptr_host.data_ptr())
        check(lib.esa_stage_masks_size(ctypes.byref(p), rp, ctypes.byref(words)),
              "esa_stage_masks_size")
        if words.value * 4 > STAGE_MASK_BUDGET:
            self._stage_masks = False
            return None
        masks = torch.empty(max(4, words.value), dtype=torch.int32, device=self.device)
        check(lib.esa_build_stage_masks(ctypes.byref(p), ctypes.c_void_p(self.row_ptr.data_ptr()),
                                        ctypes.c_void_p(self.col_idx.data_ptr()), rp,
                                        ctypes.c_void_p(masks.data_ptr()), masks.numel(),
                                        _stream(self.device)), "esa_build_stage_masks")
        self._stage_masks = masks
        return masks

    def tiles_for(self, q_len: int) -> int:
        """Active tiles over the query blocks a q_len-row prefill visits,
        summed over heads (one batch element); cached per q_len (the kernel
        choice asks on every forward)."""
        got = self._tiles_for.get(int(q_len))
        if got is not None:
            return got
        nq = (q_len + self.pattern.block_m - 1) // self.pattern.block_m
        rp = self.row_ptr_host.view(-1)[:-1].view(self.pattern.num_heads, self.num_qblocks)
        nxt = self.row_ptr_host.view(-1)[1:].view(self.pattern.num_heads, self.num_qblocks)
        got = int((nxt[:, :nq] - rp[:, :nq]).sum())
        self._tiles_for[int(q_len)] = got
        return got

    def block_cumsum(self) -> torch.Tensor:
        """float64 ``[nqb + 1]``: blocks listed for query blocks 0 .. i - 1,
        summed over heads (one batch element); host, cached."""
        if self._block_cum is None:
            H = self.pattern.num_heads
            rp = self.row_ptr_host.to(torch.int64)
            per = (rp[1:] - rp[:-1]).view(H, self.num_qblocks).sum(0).double()
            self._block_cum = torch.cat([torch.zeros(1, dtype=torch.float64), per.cumsum(0)])
        return self._block_cum

    def positions(self, row0: int, q_len: int) -> torch.Tensor:
        """int64 ``arange(row0, q_len)`` on the layout's device, cached."""
        key = (int(row0), int(q_len))
        got = self._positions.get(key)
        if got is None:
            got = torch.arange(row0, q_len, dtype=torch.int64, device=self.device)
            self._positions[key] = got
        return got

    def schedule(self, q_len: int, batch: int) -> Tuple[torch.Tensor, int]:
        key = (int(q_len), int(batch))
        got = self._schedules.get(key)
        if got is not None:
            return got
        lib = load()
        n = ctypes.c_int64()
        rp = ctypes.c_void_p(self.row_ptr_host.data_ptr())
        check(lib.esa_plan_schedule(ctypes.byref(self.pattern), rp, q_len, batch, None, 0,
                                    ctypes.byref(n)), "esa_plan_schedule")
        cap = max(1, n.value)
        items = torch.empty(cap, dtype=torch.int32)
        check(lib.esa_plan_schedule(ctypes.byref(self.pattern), rp, q_len, batch,
                                    ctypes.c_void_p(items.data_ptr()), cap, ctypes.byref(n)),
              "esa_plan_schedule")
        got = (items.to(self.device), n.value)
        self._schedules[key] = got
        return got


    def bwd_plan(self, q_len: int, batch: int, num_kv_heads: int) -> Tuple[torch.Tensor, ...]:
        """(tile_row, kv_ptr, kv_tiles, kv_items, num_kv_items) of esa_plan_bwd on
        the device, cached per (q_len, batch, kv heads)."""
        key = (int(q_len), int(batch), int(num_kv_heads))
        got = self._bwd_plans.get(key)
        if got is not None:
            return got
        lib = load()
        if self._col_idx_host is None:
            self._col_idx_host = self.col_idx[:max(self.num_tiles, 1)].cpu()
        rp = ctypes.c_void_p(self.row_ptr_host.data_ptr())
        ci = ctypes.c_void_p(self._col_idx_host.data_ptr())
        nt, ni = ctypes.c_int64(), ctypes.c_int64()
        check(lib.esa_plan_bwd(ctypes.byref(self.pattern), rp, ci, q_len, batch, num_kv_heads,
                               None, None, None, 0, None, 0, ctypes.byref(nt), ctypes.byref(ni)),
              "esa_plan_bwd")
        nkb = self.num_kblocks
        tile_row = torch.empty(max(self.num_tiles, 1), dtype=torch.int32)
        kv_ptr = torch.empty(num_kv_heads * nkb + 1, dtype=torch.int32)
        kv_tiles = torch.empty(max(nt.value, 1), dtype=torch.int32)
        kv_items = torch.empty(max(ni.value, 1), dtype=torch.int32)
        check(lib.esa_plan_bwd(ctypes.byref(self.pattern), rp, ci, q_len, batch, num_kv_heads,
                               ctypes.c_void_p(tile_row.data_ptr()),
                               ctypes.c_void_p(kv_ptr.data_ptr()),
                               ctypes.c_void_p(kv_tiles.data_ptr()), kv_tiles.numel(),
                               ctypes.c_void_p(kv_items.data_ptr()), kv_items.numel(),
                               ctypes.byref(nt), ctypes.byref(ni)), "esa_plan_bwd")
        got = (tile_row.to(self.device), kv_ptr.to(self.device), kv_tiles.to(self.device),
               kv_items.to(self.device), ni.value)
        self._bwd_plans[key] = got
        return got

    def mask_tiles(self, q_len: int) -> int:
        """Tiles whose masks a backward over q_len rows reads: the end of the
        last head's tiles among the query blocks below ceil(q_len / 128)."""
        nq = (int(q_len) + self.pattern.block_m - 1) // self.pattern.block_m
        return int(self.row_ptr_host[(self.pattern.num_heads - 1) * self.num_qblocks + nq])

    def tile_masks(self, q_len: int) -> torch.Tensor:
        """Key-major masks of the active tiles for q_len query rows
        (esa_build_tile_masks), 2 KB per tile of the query blocks q_len
        covers; cached for the last MASK_CACHE values of q_len."""
        got = self._masks.get(int(q_len))
        if got is not None:
            return got
        n = max(self.mask_tiles(q_len), 1) * 512
        masks = torch.empty(n, dtype=torch.int32, device=self.device)
        check(load().esa_build_tile_masks(ctypes.byref(self.pattern),
                                          ctypes.c_void_p(self.row_ptr.data_ptr()),
                                          ctypes.c_void_p(self.col_idx.data_ptr()),
                                          ctypes.c_void_p(self.row_ptr_host.data_ptr()), q_len,
                                          ctypes.c_void_p(masks.data_ptr()), n,
                                          _stream(self.device)), "esa_build_tile_masks")
        self._masks[int(q_len)] = masks
        return masks


def _fwd_args(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
              o_strides: Tuple[int, int, int], lse: Optional[torch.Tensor],
              scaling: float) -> EsaFwdArgs:
    B, H, Lq, D = q.shape
    a = EsaFwdArgs()
    a.dtype = _dtype_code(q.dtype)
    a.batch, a.num_heads, a.num_kv_heads = B, H, k.shape[1]
    a.q_len, a.kv_len, a.head_dim = Lq, k.shape[2], D
    a.q = q.data_ptr()
    a.q_stride_b, a.q_stride_h, a.q_stride_s = q.stride()[:3]
    a.k = k.data_ptr()
    a.k_stride_b, a.k_stride_h, a.k_stride_s = k.stride()[:3]
    a.v = v.data_ptr()
    a.v_stride_b, a.v_stride_h, a.v_stride_s = v.stride()[:3]
    a.o = o.data_ptr()
    a.o_stride_b, a.o_stride_h, a.o_stride_s = o_strides
    if lse is not None:
        a.lse = lse.data_ptr()
        a.lse_stride_b, a.lse_stride_h = lse.stride(0), lse.stride(1)
    else:
        a.lse = None
    a.sm_scale = float(scaling)
    return a


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    _require_gpu(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D [B, heads, seq, head_dim]")
    if k.shape != v.shape:
        raise ValueError(f"key {tuple(k.shape)} and value {tuple(v.shape)} shapes differ")
    if q.shape[0] != k.shape[0] or q.shape[3] != k.shape[3]:
        raise ValueError(f"query {tuple(q.shape)} and key {tuple(k.shape)} disagree on batch "
                         "or head_dim")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k and v must share one dtype")
    if q.shape[1] % k.shape[1] != 0:
        raise ValueError(f"query heads ({q.shape[1]}) must be divisible by key/value heads "
                         f"({k.shape[1]})")


# input types the MFMA prefill kernels take (others run the per-row gather)
MFMA_DTYPES = (torch.bfloat16, torch.float16)

# Measured crossovers (MI355X) between the band and the tile kernels: the
# band kernels cost about the same per 16-row group at every layer, the tile
# kernels about the same per staged 64 x 32 block, and the band kernel is the
# faster one once a group's rows stage more than this many blocks.  Forward
# (tile kernel with per-stage masks, 128 x 64 stages), over every dilated
# layer of B=1 H=32 L=8192 and 16384, B=4 H=32 L=4096, B=8 H=16 L=4096,
# B=2 H=16 L=16384 and, at D = 64, B=4 H=16 L=8192 and B=4 H=32 L=4096: at
# D = 128 the tile kernel is faster up to 15.5 blocks per group (by 5%), the
# band kernel at 18.7 (by 6%), the two within 2% at 19.0 (L=16384 layer 2);
# at D = 64 the tile kernel is faster up to 11.9 (by 10%), the band kernel
# from 14.0 (by 4-5%; tied at 14.4).  Backward, each half on its own (all
# four dQ / dK-dV pairs timed at every dilated layer of B=1 H=32 L=8192 with
# 32 and 8 kv heads, B=8 H=16 L=4096, B=4 H=32/8 L=4096, B=4 H=16 L=8192
# with 16 and 4 kv heads and B=2 H=16 L=16384): at D = 128 both halves
# switch between 14.4 and 18.7; at D = 64 the tile dQ is faster up to 11.9
# (within 1% with 8 kv heads), the band dQ from 14.0 (by 3-5%); the tile
# dK/dV up to 15.5 (by 6-17%), the band dK/dV from 18.7.
BAND_CROSSOVER = {128: 18.5, 64: 13.0}
BWD_DQ_CROSSOVER = {128: 16.5, 64: 13.0}
BWD_DKDV_CROSSOVER = {128: 16.5, 64: 17.0}


# cache_position calls with at least this many query rows (a chunked
# prefill) run the band kernel at their positions; fewer (decode) the per-row
# gather kernel
BAND_POSITION_MIN_ROWS = 32
# ... except at a dilated layer when the call has at most this many (batch,
# head, row) units at head_dim 128 (scaled by 128 / head_dim: the gather's
# cost per unit follows the row bytes): a grid under one round takes the band
# kernel one group's walk over its 64 bands (split over two waves there:
# about 19 us at D = 128, 15 us at D = 64), while the per-row gather costs
# about 5 us plus 4.5 us per 1024 units at D = 128.  Same box, the last rows
# of L=32768 at layers 4 and 7, gather against band: H=32 D=128, B=1, 32 /
# 64 / 96 / 128 rows 9 / 12-14 / 18-19 / 21-24 us against 19 / 19 / 19-20 /
# 20-21; B=4, 32 rows 21-23 against 19-21.  H=16 D=64, B=1 up to 256 rows
# 9-14 against 15-16; B=4, 96 rows (6144 units) 16-18 against 17-19, 128
# rows 19-22 against 18-21.  At layer 0 the band entry point runs the window
# kernel, 10 us from 32 rows on, faster than the gather at every size but
# B=1 with 32 rows.
BAND_POSITION_MIN_UNITS = 3072


def band_head_dim(head_dim: int) -> bool:
    """Head dims the band forward runs on MFMA: 64, 128 and 256, and any
    other multiple of 8 up to 256 through the next of them with zero
    padding (the tile kernels and the MFMA backward take 64 and 128)."""
    return 8 <= head_dim <= 256 and head_dim % 8 == 0


def _band_beats_tile(layout: ElasticLayout, q_len: int, batch: int, head_dim: int,
                     crossover: Dict[int, float]) -> bool:
    p = layout.pattern
    if p.attention_length > 64 or head_dim not in crossover or p.seq_len >= (1 << 24):
        return False  # the band kernels need attention_length <= 64 and kv_len < 2^24
    groups = batch * p.num_heads * ((q_len + 15) // 16)
    staged = batch * layout.stages().tiles_for(q_len)
    return staged > crossover[head_dim] * groups


def prefill_kernel(layout: ElasticLayout, q_len: int, batch: int, head_dim: int) -> str:
    """"band" or "tile": the faster prefill kernel for this pattern and shape
    (the band kernel needs attention_length <= 64 and kv_len < 2^24; at head
    dims other than 64 and 128 only the band kernel runs)."""
    p = layout.pattern
    band_ok = band_head_dim(head_dim) and p.attention_length <= 64 and p.seq_len < (1 << 24)
    if head_dim not in BAND_CROSSOVER and band_ok:
        return "band"
    if p.layer_idx == 0 and band_ok:
        # interpolation weight 0, a sliding window: the band entry point runs
        # the window kernel, which stages each key of a 32-row group once
        # (measured against the tile kernel: B=1 H=32 L=32768 D=128 0.240 vs
        # 0.246 ms, B=8 H=16 L=4096 D=64 0.050 vs 0.055, B=1 H=8 L=131072
        # 0.251 vs 0.254, B=1 H=32 L=8192 within 1%; since then the window
        # kernel's groups load each shared pair at the same step: 0.237,
        # 0.048, 0.244 and 0.050 ms)
        return "band"
    return "band" if _band_beats_tile(layout, q_len, batch, head_dim, BAND_CROSSOVER) else "tile"


# A prefill split by rows: the tile kernel on rows [0, R), the band kernel
# (at positions R ..) on [R, q_len).  A dilated layer's low rows list few
# blocks (narrow windows: the tile kernel's work grows with them) and its
# high rows many (the band kernel's work per 16-row group is about fixed),
# so where both kernels are close over the whole prefill, each taking its
# own rows beats either.  Cost model (ms) fitted to the two kernels timed on
# row ranges at every split in 1/8 steps of B=8 H=16 L=4096 D=64 and B=1
# H=32 L=8192 / 32768 D=128, layers 2, 4 and 7 (MI355X): a x (64 x 32
# blocks the tile rows list) + (b0 + b1 alpha) x (16-row groups of the band
# rows) + per-launch overheads (alpha = the layer's interpolation weight:
# later layers have narrower bands and cheaper groups).  The split is taken
# only where the model puts it SPLIT_MIN_GAIN below the better single
# kernel.  Measured with the split the model picks: B=8 H=16 L=4096 D=64
# layer 7 (rows from 1664) 0.258 vs 0.281 ms for the band kernel alone,
# B=1 H=32 L=8192 D=128 layer 4 (from 3584) 0.287 vs 0.308 ms, B=1 H=32
# L=32768 layer 2 (from 7552) 1.281 vs 1.387 ms; L=8192 layer 7, where the
# model predicts 7%, 0.277 vs 0.271 ms (the band kernel alone stays there).
# The two launches run in sequence: on two streams they were 1-5% slower.
SPLIT_MODEL = {64: (6.66e-7, 1.048e-5, -1.916e-6, 0.0126, 0.0244),
               128: (1.157e-6, 2.118e-5, -3.321e-6, 0.0124, 0.0167)}
SPLIT_MIN_GAIN = 0.08


def prefill_split(layout: ElasticLayout, q_len: int, batch: int, head_dim: int) -> int:
    """The row R from which the band kernel takes a prefill's rows, the tile
    kernel taking rows [0, R): q_len for the tile kernel alone, 0 for the
    band kernel alone, else a multiple of 128 (see SPLIT_MODEL); cached per
    shape."""
    key = (int(q_len), int(batch), int(head_dim))
    got = layout._splits.get(key)
    if got is not None:
        return got
    single = prefill_kernel(layout, q_len, batch, head_dim)
    R = 0 if single == "band" else q_len
    p = layout.pattern
    if head_dim in SPLIT_MODEL and p.layer_idx > 0 and q_len >= 256 and \
            p.attention_length <= 64 and p.seq_len < (1 << 24):
        a, b0, b1, o_tile, o_band = SPLIT_MODEL[head_dim]
        alpha = p.layer_idx / (p.num_hidden_layers - 1) if p.num_hidden_layers > 1 else 0.0
        st = layout.stages()
        cum = st.block_cumsum()
        bm = st.pattern.block_m
        per_group = (b0 + b1 * alpha) * batch * p.num_heads
        rows = torch.arange(128, q_len, 128, dtype=torch.int64)
        if rows.numel() > 0:
            tile = a * batch * cum[torch.clamp((rows + bm - 1) // bm, max=cum.numel() - 1)]
            band = per_group * ((q_len - rows + 15) // 16).double()
            cost = tile + band + o_tile + o_band
            i = int(torch.argmin(cost))
            tile_only = a * batch * float(cum[min((q_len + bm - 1) // bm, cum.numel() - 1)]) + o_tile
            band_only = per_group * ((q_len + 15) // 16) + o_band
            if float(cost[i]) <= (1.0 - SPLIT_MIN_GAIN) * min(tile_only, band_only):
                R = int(rows[i])
    layout._splits[key] = R
    return R


def bwd_kernels(layout: ElasticLayout, q_len: int, batch: int, head_dim: int
                ) -> Tuple[str, str]:
    """("band" | "tile", "band" | "tile"): the faster dQ and dK/dV kernels for
    this pattern and shape, each half switching to its band kernel at its own
    measured crossover (BWD_DQ_CROSSOVER, BWD_DKDV_CROSSOVER)."""
    p = layout.pattern
    if (p.layer_idx == 0 and head_dim in BWD_DQ_CROSSOVER and p.attention_length <= 64
            and p.seq_len < (1 << 24)):
        # interpolation weight 0, a sliding window: both band kernels walk the
        # window's keys and rows directly (measured against tile / tile: B=1
        # H=32 L=32768 D=128 0.803 vs 0.952 ms, B=1 H=32 L=8192 0.225 vs
        # 0.261, B=8 H=16 L=4096 D=64 0.220 vs 0.245, B=1 H=8 L=131072 0.810
        # vs 0.962; band / band is also faster than either mixed pair)
        return "band", "band"
    dq = _band_beats_tile(layout, q_len, batch, head_dim, BWD_DQ_CROSSOVER)
    dkdv = _band_beats_tile(layout, q_len, batch, head_dim, BWD_DKDV_CROSSOVER)
    return "band" if dq else "tile", "band" if dkdv else "tile"


def elastic_attention_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          layout: ElasticLayout, scaling: float, return_lse: bool = True,
                          out: Optional[torch.Tensor] = None, key_block: Optional[int] = None,
                          query_block: Optional[int] = None, kernel: str = "auto",
                          stage_masks: bool = True
                          ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Prefill forward over the elastic pattern (query row r is position r).

    Returns ``o`` as ``[B, Lq, H, D]`` (so ``o.view(B, Lq, H * D)`` is the
    module output, :761-763) and, if asked, ``lse`` float32 ``[B, H, Lq]``.

    ``kernel``: "tile" is the block-sparse MFMA kernel over ``layout``;
    "band" the band-gathered kernel (:func:`elastic_attention_band`); "auto"
    takes the faster for the shape (:func:`prefill_kernel`).  Both agree to
    bf16 rounding.  For the tile kernel the staging unit is ``query_block``
    x ``key_block``: (64, 32) gives each workgroup of two waves 64 query
    rows and stages K/V in 32-key blocks from the pattern's 64 x 32 layout;
    (128, 64) gives four waves 128 rows and 64-key stages (halves of 128-key
    tiles no row needs are skipped); (128, 128) stages whole 128-key tiles of
    ``layout``.  All tile variants give the same output bit for bit.  By
    default (128, 64): at layer 0 (a sliding window) 1.5 staged keys per row
    instead of 2, 4-8% faster at four of the five measured shapes; at the
    dilated layers, with per-stage masks, 2-11% faster than (64, 32) at every
    shape and layer where the tile kernel is the faster prefill kernel.
    ``stage_masks``: at dilated layers the
    kernel loads each row's valid keys per stage from masks built once per
    layout (:meth:`ElasticLayout.stage_masks`, within STAGE_MASK_BUDGET)
    instead of walking the row's index list; the output is the same bit for
    bit.
    """
    _check_qkv(q, k, v)
    return _prefill_fwd(q, k, v, layout, scaling, return_lse, out, key_block, query_block,
                        kernel, stage_masks)


def _prefill_fwd(q, k, v, layout, scaling, return_lse, out, key_block, query_block, kernel,
                 stage_masks):
    """elastic_attention_fwd after its q / k / v checks (the module, which
    checks them itself, calls this directly)."""
    B, H, Lq, D = q.shape
    if kernel not in ("auto", "tile", "band"):
        raise ValueError(f"kernel must be 'auto', 'tile' or 'band', got {kernel!r}")
    split = Lq
    if kernel == "auto":
        split = prefill_split(layout, Lq, B, D)
        kernel = "band" if split == 0 else "tile"
        if out is not None and out.data_ptr() % 16 != 0:
            kernel, split = "tile", Lq
    if kernel == "band":
        return elastic_attention_band(q, k, v, layout.pattern, scaling, return_lse, out)
    q, k, v = _prep(q, 8), _prep(k, 8), _prep(v, 8)
    o = out if out is not None else torch.empty(B, Lq, H, D, dtype=q.dtype, device=q.device)
    lse = torch.empty(B, H, Lq, dtype=torch.float32, device=q.device) if return_lse else None
    if 0 < split < Lq:
        # rows [split, Lq) by the band kernel at their positions, then rows
        # [0, split) by the tile kernel below (views of the same o and lse)
        _band_launch(q[:, :, split:], k, v, o[:, split:], None if lse is None else
                     lse[:, :, split:], layout.pattern, scaling, layout.positions(split, Lq))
        q, o_all, lse_all = q[:, :, :split], o, lse
        o = o[:, :split]
        lse = None if lse is None else lse[:, :, :split]
        Lq = split
    else:
        o_all, lse_all = o, lse
    if query_block is None and key_block is None:
        query_block, key_block = 128, 64
    if (query_block, key_block) not in ((128, 64), (128, 128), (64, 32)):
        raise ValueError(f"(query_block, key_block) must be (128, 64), (128, 128) or (64, 32), "
                         f"got ({query_block}, {key_block})")
    if B == 0 or Lq == 0:
        return o_all, lse_all  # no rows: nothing to launch (empty tensors may have no address)
    st = layout if (query_block, key_block) == (128, 128) else layout.stages(key_block,
                                                                             query_block)
    items, n = st.schedule(Lq, B)
    # layer 0 rows are contiguous runs: the kernel sets them without a walk
    # (measured: with masks 5-8% slower at B=8 H=16 L=4096 and B=1 H=32
    # L=8192, within 2% elsewhere); whole-tile staging walks
    use = stage_masks and st.pattern.layer_idx > 0 and st.pattern.block_n != 128
    masks = st.stage_masks() if use else None
    a = _fwd_args(q, k, v, o, (o.stride(0), o.stride(2), o.stride(1)), lse, scaling)
    check(load().esa_elastic_fwd(ctypes.byref(a), ctypes.byref(st.pattern),
                                 ctypes.c_void_p(st.row_ptr.data_ptr()),
                                 ctypes.c_void_p(st.col_idx.data_ptr()),
                                 ctypes.c_void_p(st.row_ptr_host.data_ptr()),
                                 ctypes.c_void_p(masks.data_ptr() if masks is not None else None),
                                 masks.numel() if masks is not None else 0,
                                 ctypes.c_void_p(items.data_ptr()), n, _stream(q.device)),
          "esa_elastic_fwd")
    return o_all, lse_all


def elastic_attention_band(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           pattern: EsaPattern, scaling: float, return_lse: bool = True,
                           out: Optional[torch.Tensor] = None,
                           positions: Optional[torch.Tensor] = None
                           ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Band-gathered MFMA forward, no layout needed: each wave takes 16 query
    rows and, for every entry j of their index lists, gathers the at most 16
    consecutive keys those rows use at entry j.  Query row r is position r,
    or ``positions[r]`` (int64 on the device, as cache_position: a chunked
    prefill's consecutive positions run as prefill groups, any other 16-row
    group through the per-row gather).  Returns ``o`` ``[B, Lq, H, D]`` and,
    if asked, ``lse`` float32 ``[B, H, Lq]``, as
    :func:`elastic_attention_fwd`."""
    _check_qkv(q, k, v)
    B, H, Lq, D = q.shape
    q, k, v = _prep(q, 8), _prep(k, 8), _prep(v, 8)
    o = out if out is not None else torch.empty(B, Lq, H, D, dtype=q.dtype, device=q.device)
    lse = torch.empty(B, H, Lq, dtype=torch.float32, device=q.device) if return_lse else None
    _band_launch(q, k, v, o, lse, pattern, scaling, positions)
    return o, lse


def _band_launch(q, k, v, o, lse, pattern, scaling, positions) -> None:
    """esa_elastic_fwd_band into o ``[B, Lq, H, D]`` (and lse) for q's rows
    (q, k, v prepared, o's rows 16-byte aligned)."""
    B, H, Lq, D = q.shape
    positions, pos_ptr = _positions_ptr(positions, Lq, q.device)
    if B == 0 or Lq == 0:
        return
    a = _fwd_args(q, k, v, o, (o.stride(0), o.stride(2), o.stride(1)), lse, scaling)
    check(load().esa_elastic_fwd_band(ctypes.byref(a), ctypes.byref(pattern), pos_ptr,
                                      _stream(q.device)), "esa_elastic_fwd_band")


def _positions_ptr(positions: Optional[torch.Tensor], q_len: int, device: torch.device):
    if positions is None:
        return None, None
    if positions.dtype != torch.int64 or positions.device != device or \
            positions.numel() != q_len:
        raise ValueError("positions must be an int64 tensor of q_len entries on q's device")
    positions = positions.contiguous()
    return positions, ctypes.c_void_p(positions.data_ptr())


def elastic_attention_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           pattern: EsaPattern, scaling: float,
                           positions: Optional[torch.Tensor] = None, return_lse: bool = True,
                           dropout_p: float = 0.0, seed: int = 0, return_weights: bool = False
                           ):
    """Per-row gather forward over the pattern (float32, bfloat16 or
    float16, any head_dim that is a multiple of 4 up to 256); query row r is
    position ``positions[r]`` (int64 on the device) or r.  Output
    ``[B, Lq, H, D]`` and, if asked, lse ``[B, H, Lq]``.

    ``dropout_p`` > 0 applies attention dropout to the probabilities (the
    naive path in training mode, :674) with keep decisions drawn from
    ``seed``; ``return_weights`` also returns the naive path's attention
    weights ``[B, H, Lq, w]`` (after dropout, :673-680) as a third value."""
    _check_qkv(q, k, v)
    return _rows_fwd(q, k, v, pattern, scaling, positions, return_lse, dropout_p, seed,
                     return_weights)


def _rows_fwd(q, k, v, pattern, scaling, positions, return_lse, dropout_p, seed,
              return_weights):
    """elastic_attention_rows after its argument checks (the module, which
    checks q, k, v itself, calls this directly)."""
    B, H, Lq, D = q.shape
    q, k, v = _prep(q, 4), _prep(k, 4), _prep(v, 4)
    o = torch.empty(B, Lq, H, D, dtype=q.dtype, device=q.device)
    need_lse = return_lse or return_weights
    lse = torch.empty(B, H, Lq, dtype=torch.float32, device=q.device) if need_lse else None
    positions, pos_ptr = _positions_ptr(positions, Lq, q.device)
    if B == 0 or Lq == 0:
        lse_out = lse if return_lse else None
        if return_weights:
            wts = torch.empty(B, H, Lq, pattern.attention_length, dtype=q.dtype,
                              device=q.device)
            return o, lse_out, wts
        return o, lse_out
    a = _fwd_args(q, k, v, o, (o.stride(0), o.stride(2), o.stride(1)), lse, scaling)
    if dropout_p > 0.0 or return_weights:
        wts = None
        opts = EsaNaiveOpts()
        opts.dropout_p = float(dropout_p)
        opts.seed = int(seed) & ((1 << 64) - 1)
        if return_weights:
            wts = torch.empty(B, H, Lq, pattern.attention_length, dtype=q.dtype, device=q.device)
            opts.weights = wts.data_ptr()
            opts.weights_stride_b, opts.weights_stride_h, opts.weights_stride_s = wts.stride()[:3]
        check(load().esa_elastic_fwd_naive(ctypes.byref(a), ctypes.byref(pattern), pos_ptr,
                                           ctypes.byref(opts), _stream(q.device)),
              "esa_elastic_fwd_naive")
        lse_out = lse if return_lse else None
        return (o, lse_out, wts) if return_weights else (o, lse_out)
    check(load().esa_elastic_fwd_rows(ctypes.byref(a), ctypes.byref(pattern), pos_ptr,
                                      _stream(q.device)), "esa_elastic_fwd_rows")
    return o, lse


def sparse_attention_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         sparse_indices: torch.Tensor, sparse_mask: torch.Tensor,
                         sm_scale: float, num_kv_groups: int
                         ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Gather forward over explicit ``[H, Lq, w]`` index lists (the reference
    operator, :241-297).  Returns ``o [B, H, Lq, D]`` (q's shape and dtype)
    and ``lse [B, H, Lq]``."""
    _check_qkv(q, k, v)
    _require_gpu(sparse_indices, sparse_mask)
    B, H, Lq, D = q.shape
    if num_kv_groups != H // k.shape[1]:
        raise ValueError(f"num_kv_groups ({num_kv_groups}) != query heads / key heads "
                         f"({H} / {k.shape[1]})")
    if sparse_indices.shape != sparse_mask.shape or sparse_indices.dim() != 3 or \
            sparse_indices.shape[0] != H or sparse_indices.shape[1] != Lq:
        raise ValueError(f"sparse_indices/sparse_mask must be [H={H}, Lq={Lq}, w]; got "
                         f"{tuple(sparse_indices.shape)} and {tuple(sparse_mask.shape)}")
    if sparse_indices.dtype not in (torch.int64, torch.int32):
        raise ValueError("sparse_indices must be int64 or int32")
    q, k, v = _prep(q, 4), _prep(k, 4), _prep(v, 4)
    idx, msk = _index_arrays(sparse_indices, sparse_mask)
    o = torch.empty(B, H, Lq, D, dtype=q.dtype, device=q.device)
    lse = torch.empty(B, H, Lq, dtype=torch.float32, device=q.device)
    if B == 0 or Lq == 0:
        return o, lse
    a = _fwd_args(q, k, v, o, (o.stride(0), o.stride(1), o.stride(2)), lse, sm_scale)
    check(load().esa_sparse_fwd(ctypes.byref(a), ctypes.c_void_p(idx.data_ptr()),
                                idx.element_size(), idx.stride(0), idx.stride(1),
                                ctypes.c_void_p(msk.data_ptr()), msk.element_size(),
                                msk.stride(0), msk.stride(1), idx.shape[2], _stream(q.device)),
          "esa_sparse_fwd")
    return o, lse


def _bwd_args(q, k, v, o, o_strides, lse, dout, dout_strides, dq, dk, dv, scaling) -> EsaBwdArgs:
    B, H, Lq, D = q.shape
    a = EsaBwdArgs()
    a.dtype = _dtype_code(q.dtype)
    a.batch, a.num_heads, a.num_kv_heads = B, H, k.shape[1]
    a.q_len, a.kv_len, a.head_dim = Lq, k.shape[2], D
    for name, t, strides in (("q", q, q.stride()[:3]), ("k", k, k.stride()[:3]),
                             ("v", v, v.stride()[:3]), ("o", o, o_strides),
                             ("dout", dout, dout_strides), ("dq", dq, dq.stride()[:3]),
                             ("dk", dk, dk.stride()[:3]), ("dv", dv, dv.stride()[:3])):
        setattr(a, name, t.data_ptr())
        for ax, st in zip("bhs", strides):
            setattr(a, f"{name}_stride_{ax}", st)
    a.lse = lse.data_ptr()
    a.lse_stride_b, a.lse_stride_h = lse.stride(0), lse.stride(1)
    a.sm_scale = float(scaling)
    return a


def _gather_workspace(a: EsaBwdArgs, w: int, device: torch.device) -> torch.Tensor:
    ws = ctypes.c_size_t()
    check(load().esa_gather_bwd_workspace_size(ctypes.byref(a), int(w), ctypes.byref(ws)),
          "esa_gather_bwd_workspace_size")
    return torch.empty(max(ws.value, 256), dtype=torch.uint8, device=device)


def elastic_attention_bwd_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                               o: torch.Tensor, lse: torch.Tensor, dout: torch.Tensor,
                               pattern: EsaPattern, scaling: float,
                               positions: Optional[torch.Tensor] = None, dropout_p: float = 0.0,
                               seed: int = 0
                               ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gather backward of :func:`elastic_attention_rows` (any dtype it takes,
    any head_dim, decode positions, dropout with the forward's seed): ``o``
    and ``dout`` ``[B, Lq, H, D]``, ``lse`` ``[B, H, Lq]``.  Returns ``dq``
    ``[B, H, Lq, D]``, ``dk`` and ``dv`` ``[B, Hkv, Lk, D]``; deterministic
    (no atomics on the gradients)."""
    _check_qkv(q, k, v)
    B, H, Lq, D = q.shape
    q, k, v = _prep(q, 4), _prep(k, 4), _prep(v, 4)
    dout = dout.to(q.dtype)
    lse = lse.contiguous()
    dq = torch.empty(B, H, Lq, D, dtype=q.dtype, device=q.device)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    if B == 0 or Lq == 0:
        return dq, dk.zero_(), dv.zero_()  # no query row reaches a key
    a = _bwd_args(q, k, v, o, (o.stride(0), o.stride(2), o.stride(1)), lse, dout,
                  (dout.stride(0), dout.stride(2), dout.stride(1)), dq, dk, dv, scaling)
    work = _gather_workspace(a, pattern.attention_length, q.device)
    positions, pos_ptr = _positions_ptr(positions, Lq, q.device)
    check(load().esa_elastic_bwd_rows(ctypes.byref(a), ctypes.byref(pattern), pos_ptr,
                                      float(dropout_p), int(seed) & ((1 << 64) - 1),
                                      ctypes.c_void_p(work.data_ptr()), work.numel(),
                                      _stream(q.device)), "esa_elastic_bwd_rows")
    return dq, dk, dv


def _index_arrays(sparse_indices: torch.Tensor, sparse_mask: torch.Tensor):
    idx = sparse_indices.contiguous()
    msk = sparse_mask
    if msk.dtype == torch.bool:
        msk = msk.to(torch.uint8)
    elif msk.dtype not in (torch.int64, torch.int32, torch.uint8):
        msk = msk.to(torch.int32)
    return idx, msk.contiguous()


def sparse_attention_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                         lse: torch.Tensor, dout: torch.Tensor, sparse_indices: torch.Tensor,
                         sparse_mask: torch.Tensor, sm_scale: float
                         ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Backward of :func:`sparse_attention_fwd` (the reference operator's
    backward, :299-339): ``o`` and ``dout`` ``[B, H, Lq, D]``.  Returns
    ``dq``, ``dk``, ``dv`` in the inputs' shapes and dtype; deterministic."""
    _check_qkv(q, k, v)
    B, H, Lq, D = q.shape
    q, k, v = _prep(q, 4), _prep(k, 4), _prep(v, 4)
    dout = dout.to(q.dtype)
    idx, msk = _index_arrays(sparse_indices, sparse_mask)
    dq = torch.empty(B, H, Lq, D, dtype=q.dtype, device=q.device)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    if B == 0 or Lq == 0:
        return dq, dk.zero_(), dv.zero_()
    a = _bwd_args(q, k, v, o, o.stride()[:3], lse.contiguous(), dout, dout.stride()[:3], dq, dk,
                  dv, sm_scale)
    work = _gather_workspace(a, idx.shape[2], q.device)
    check(load().esa_sparse_bwd(ctypes.byref(a), ctypes.c_void_p(idx.data_ptr()),
                                idx.element_size(), idx.stride(0), idx.stride(1),
                                ctypes.c_void_p(msk.data_ptr()), msk.element_size(),
                                msk.stride(0), msk.stride(1), idx.shape[2],
                                ctypes.c_void_p(work.data_ptr()), work.numel(),
                                _stream(q.device)), "esa_sparse_bwd")
    return dq, dk, dv


def elastic_attention_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                          lse: torch.Tensor, dout: torch.Tensor, layout: ElasticLayout,
                          scaling: float, dq_kernel: str = "auto", dkdv_kernel: str = "auto",
                          noalloc: bool = False, stage_masks: bool = True
                          ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """MFMA backward of ``elastic_attention_fwd`` (prefill, bf16 or fp16).

    ``noalloc``: call ``esa_elastic_bwd_noalloc`` (the library's per-device
    workspace array, no workspace allocation) instead of ``esa_elastic_bwd``.
    ``stage_masks``: at dilated layers the block-sparse dQ loads each row's
    valid keys per tile from the layout's row masks
    (:meth:`ElasticLayout.stage_masks`, within STAGE_MASK_BUDGET) instead of
    walking the row's index list; the gradients are the same bit for bit.

    ``o`` and ``dout`` are ``[B, Lq, H, D]`` (the forward's output layout),
    ``lse`` float32 ``[B, H, Lq]``.  Returns ``dq`` ``[B, H, Lq, D]`` and
    ``dk``, ``dv`` ``[B, Hkv, Lk, D]``: the gradients the reference's
    ElasticSparseAttentionFunction.backward returns (:299-339), computed
    without atomics.  ``dq_kernel`` and ``dkdv_kernel``: "band" computes that
    half with a band-gathered kernel (dQ row-major, dK/dV key-major), "tile"
    block-sparse over the layout, "auto" as :func:`bwd_kernels` picks.
    """
    _check_qkv(q, k, v)
    B, H, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    q, k, v = _prep(q, 8), _prep(k, 8), _prep(v, 8)
    o = _prep(o, 8)
    dout = _prep(dout, 8)
    lse = lse.contiguous()
    dq = torch.empty_like(q)
    dk = torch.empty(B, Hkv, Lk, D, dtype=k.dtype, device=k.device)
    dv = torch.empty(B, Hkv, Lk, D, dtype=v.dtype, device=v.device)
    for name, val in (("dq_kernel", dq_kernel), ("dkdv_kernel", dkdv_kernel)):
        if val not in ("auto", "tile", "band"):
            raise ValueError(f"{name} must be 'auto', 'tile' or 'band', got {val!r}")
    if B == 0 or Lq == 0:
        return dq, dk.zero_(), dv.zero_()  # no query row reaches a key
    a = _bwd_args(q, k, v, o, (o.stride(0), o.stride(2), o.stride(1)), lse, dout,
                  (dout.stride(0), dout.stride(2), dout.stride(1)), dq, dk, dv, scaling)
    lib = load()
    work = None
    if noalloc:
        init_device(q.device)
    else:
        ws = ctypes.c_size_t()
        check(lib.esa_bwd_workspace_size(ctypes.byref(a), ctypes.byref(ws)),
              "esa_bwd_workspace_size")
        work = torch.empty(max((ws.value + 3) // 4, 4), dtype=torch.float32, device=q.device)
    auto_dq, auto_dkdv = bwd_kernels(layout, Lq, B, D)
    dq_kernel = auto_dq if dq_kernel == "auto" else dq_kernel
    dkdv_kernel = auto_dkdv if dkdv_kernel == "auto" else dkdv_kernel
    vp = ctypes.c_void_p

    def ptr(t):
        return vp(t.data_ptr() if t is not None else None)

    # a band half takes no work list (its kernel covers every row group or
    # key block), and no layout arrays when both halves are band-gathered
    items, n_items = (None, 0) if dq_kernel == "band" else layout.schedule(Lq, B)
    q_masks = None
    if dq_kernel == "tile" and stage_masks and layout.pattern.layer_idx > 0:
        q_masks = layout.stage_masks()
    if dkdv_kernel == "band":
        tile_row = kv_ptr = kv_tiles = kv_items = masks = None
        n_kv = 0
    else:
        tile_row, kv_ptr, kv_tiles, kv_items, n_kv = layout.bwd_plan(Lq, B, Hkv)
        masks = layout.tile_masks(Lq)
    def words(t):
        return t.numel() if t is not None else 0

    if noalloc:
        check(lib.esa_elastic_bwd_noalloc(ctypes.byref(a), ctypes.byref(layout.pattern),
                                          ptr(layout.row_ptr), ptr(layout.col_idx),
                                          ptr(layout.row_ptr_host), ptr(items), n_items,
                                          ptr(tile_row), ptr(kv_ptr), ptr(kv_tiles),
                                          ptr(kv_items), n_kv, ptr(masks), words(masks),
                                          ptr(q_masks), words(q_masks), _stream(q.device)),
              "esa_elastic_bwd_noalloc")
    else:
        check(lib.esa_elastic_bwd(ctypes.byref(a), ctypes.byref(layout.pattern),
                                  ptr(layout.row_ptr), ptr(layout.col_idx),
                                  ptr(layout.row_ptr_host), ptr(items), n_items, ptr(tile_row),
                                  ptr(kv_ptr), ptr(kv_tiles), ptr(kv_items), n_kv, ptr(masks),
                                  words(masks), ptr(q_masks), words(q_masks), ptr(work),
                                  work.numel() * 4, _stream(q.device)),
              "esa_elastic_bwd")
    return dq, dk, dv


class _ElasticTileAttention(torch.autograd.Function):
    """Prefill forward (either kernel) with the MFMA backward (kernels as
    :func:`bwd_kernels` picks):
    ``apply(q, k, v, layout, scaling, kernel) -> o [B, Lq, H, D]``."""

    @staticmethod
    def forward(ctx, q, k, v, layout, scaling, kernel="auto"):
        o, lse = elastic_attention_fwd(q, k, v, layout, scaling, return_lse=True, kernel=kernel)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.layout = layout
        ctx.scaling = scaling
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = elastic_attention_bwd(q, k, v, o, lse, do, ctx.layout, ctx.scaling)
        return dq, dk, dv, None, None, None


class _ElasticBandRowsAttention(torch.autograd.Function):
    """The band forward at cache_position rows (chunked prefill; positions
    None: rows 0 .. Lq - 1), or at a head_dim the MFMA backward does not
    take, with the gather backward at the same positions:
    ``apply(q, k, v, pattern, scaling, positions) -> o [B, Lq, H, D]``."""

    @staticmethod
    def forward(ctx, q, k, v, pattern, scaling, positions):
        o, lse = elastic_attention_band(q, k, v, pattern, scaling, return_lse=True,
                                        positions=positions)
        ctx.save_for_backward(q, k, v, o, lse, positions)
        ctx.pattern, ctx.scaling = pattern, scaling
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, positions = ctx.saved_tensors
        dq, dk, dv = elastic_attention_bwd_rows(q, k, v, o, lse, do, ctx.pattern, ctx.scaling,
                                                positions)
        return dq, dk, dv, None, None, None


class ElasticSparseAttentionFunction(torch.autograd.Function):
    """The reference's operator (:235-339): ``apply(q, k, v, sparse_indices,
    sparse_mask, sm_scale, num_kv_groups) -> o [B, H, Lq, D]``, with its
    backward (dq, dk, dv; none for the index arguments) by the gather
    backward kernels, deterministic where the reference uses atomics."""

    @staticmethod
    def forward(ctx, q, k, v, sparse_indices, sparse_mask, sm_scale, num_kv_groups):
        o, lse = sparse_attention_fwd(q, k, v, sparse_indices, sparse_mask, sm_scale,
                                      num_kv_groups)
        ctx.save_for_backward(q, k, v, o, lse, sparse_indices, sparse_mask)
        ctx.sm_scale = sm_scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, idx, msk = ctx.saved_tensors
        dq, dk, dv = sparse_attention_bwd(q, k, v, o, lse, do, idx, msk, ctx.sm_scale)
        return dq, dk, dv, None, None, None, None


class _ElasticRowsAttention(torch.autograd.Function):
    """The per-row gather forward over the pattern with the gather backward:
    ``apply(q, k, v, pattern, scaling, positions, dropout_p, seed,
    with_weights) -> (o [B, Lq, H, D], weights)``; weights is the naive
    path's ``[B, H, Lq, w]`` (not differentiable) or an empty tensor."""

    @staticmethod
    def forward(ctx, q, k, v, pattern, scaling, positions, dropout_p, seed, with_weights):
        got = elastic_attention_rows(q, k, v, pattern, scaling, positions, return_lse=True,
                                     dropout_p=dropout_p, seed=seed,
                                     return_weights=with_weights)
        o, lse = got[0], got[1]
        wts = got[2] if with_weights else o.new_empty(0)
        ctx.save_for_backward(q, k, v, o, lse, positions)
        ctx.pattern, ctx.scaling, ctx.dropout_p, ctx.seed = pattern, scaling, dropout_p, seed
        ctx.mark_non_differentiable(wts)
        return o, wts

    @staticmethod
    def backward(ctx, do, _dw):
        q, k, v, o, lse, positions = ctx.saved_tensors
        dq, dk, dv = elastic_attention_bwd_rows(q, k, v, o, lse, do, ctx.pattern, ctx.scaling,
                                                positions, ctx.dropout_p, ctx.seed)
        return dq, dk, dv, None, None, None, None, None, None


class ElasticSparseAttention(nn.Module):
    """Drop-in for the reference's ElasticSparseAttention (:345-765), on HIP.

    Args mirror :375-386.  ``scaling = head_dim ** -0.5`` (:444),
    ``num_kv_groups = H // Hkv`` (:442); query head h reads kv head
    ``h // num_kv_groups`` (:89).
    """

    def __init__(self, layer_idx: int, num_hidden_layers: int, num_attention_heads: int,
                 head_dim: int, attention_length: int, max_seq_len: int,
                 num_key_value_heads: Optional[int] = None, attention_dropout: float = 0.0,
                 implementation: str = "triton"):
        super().__init__()
        valid_implementations = ["triton", "naive", "dense"]
        if implementation not in valid_implementations:                   # :412-417
            raise ValueError(
                f"Invalid implementation '{implementation}'. Must be one of "
                f"{valid_implementations}.")
        self.layer_idx = layer_idx
        self.num_hidden_layers = num_hidden_layers
        self.num_attention_heads = num_attention_heads
        self.head_dim = head_dim
        self.attention_length = attention_length
        self.attention_dropout = attention_dropout
        self.implementation = implementation
        self.max_seq_len = max_seq_len
        self.num_key_value_heads = (num_key_value_heads if num_key_value_heads is not None
                                    else num_attention_heads)
        if self.num_attention_heads % self.num_key_value_heads != 0:      # :435-441
            raise ValueError(
                f"`num_attention_heads` ({self.num_attention_heads}) must be divisible by "
                f"`num_key_value_heads` ({self.num_key_value_heads}) for GQA.")
        self.num_kv_groups = self.num_attention_heads // self.num_key_value_heads  # :442
        self.scaling = self.head_dim ** -0.5                                  # :444
        self.pattern = make_pattern(max_seq_len, attention_length, layer_idx,
                                    num_hidden_layers, num_attention_heads)
        self._layouts: Dict[torch.device, ElasticLayout] = {}
        # The reference's cached index buffers (:454-468), registered the same
        # way (non-persistent, so they follow module.to() and stay out of the
        # state dict).  The kernels regenerate indices and never read them, so
        # they start out None and are built on first access, by the HIP
        # builders, on the device the module lives on: "dense" gets
        # full_attention_mask, the others the index set and its mask, as the
        # reference registers them.  An empty anchor buffer records that
        # device.
        self.register_buffer("_anchor", torch.empty(0), persistent=False)
        self.register_buffer("sparse_attention_indices", None, persistent=False)
        self.register_buffer("sparse_causal_mask", None, persistent=False)
        self.register_buffer("full_attention_mask", None, persistent=False)
        # bf16 prefill kernel: "auto" (the faster for the shape), "band" or "tile"
        self.prefill_kernel = "auto"

    _LAZY_BUFFERS = ("sparse_attention_indices", "sparse_causal_mask", "full_attention_mask")

    def __getattr__(self, name: str):
        buffers = self.__dict__.get("_buffers", {})
        if name in ElasticSparseAttention._LAZY_BUFFERS and name in buffers:
            if buffers[name] is None:
                self._materialise(name)
            return buffers[name]
        return super().__getattr__(name)

    def _materialise(self, name: str) -> None:
        """Builds the reference's buffer ``name`` on the module's device, if
        this implementation registers it (:454-468); leaves it None
        otherwise."""
        buffers = self.__dict__["_buffers"]
        device = buffers["_anchor"].device
        L = self.max_seq_len
        if self.implementation == "dense":
            if name == "full_attention_mask":
                buffers[name] = self._create_full_sparse_mask(L, device)
        elif name != "full_attention_mask":
            idx, msk = self._create_elastic_sparse_indices(L, device)
            buffers["sparse_attention_indices"] = idx
            buffers["sparse_causal_mask"] = msk

    @staticmethod
    def _builder_device(device: torch.device) -> torch.device:
        """The GPU the HIP builders run on for a buffer wanted on ``device``
        (the current GPU for a CPU-resident module: the product has no CPU
        path, so the result is copied there)."""
        device = torch.device(device)
        if device.type == "cuda":
            return device if device.index is not None else torch.device(
                "cuda", torch.cuda.current_device())
        if not torch.cuda.is_available():
            raise RuntimeError("the elastic index builders run on the GPU through libesa.so "
                               "(HIP); no GPU is available")
        return torch.device("cuda", torch.cuda.current_device())

    def _create_elastic_sparse_indices(self, seq_len: int, device: torch.device
                                       ) -> Tuple[torch.Tensor, torch.Tensor]:
        """``(indices, mask)``, int64 ``[H, seq_len, w]`` on ``device``, as the
        reference's method of this name returns them (:470-535): masked
        entries have index 0 and mask 0.  Built by the HIP index builder
        (esa_build_indices, bit-exact)."""
        dev = self._builder_device(device)
        pat = make_pattern(seq_len, self.attention_length, self.layer_idx,
                           self.num_hidden_layers, self.num_attention_heads)
        idx, msk = build_indices(pat, dev, torch.int64)
        return idx.to(device), msk.to(device)

    def _create_full_sparse_mask(self, seq_len: int, device: torch.device) -> torch.Tensor:
        """bool ``[1, H, seq_len, seq_len]`` on ``device``: True where the
        query row lists the key among its valid entries, as the reference's
        method of this name returns it (:537-572).  Built by the HIP
        dense-mask builder (esa_build_dense_mask) from the same index set."""
        dev = self._builder_device(device)
        pat = make_pattern(seq_len, self.attention_length, self.layer_idx,
                           self.num_hidden_layers, self.num_attention_heads)
        H = self.num_attention_heads
        mask = torch.empty(1, H, seq_len, seq_len, dtype=torch.bool, device=dev)
        if seq_len > 0:
            check(load().esa_build_dense_mask(ctypes.byref(pat), 0, seq_len, seq_len,
                                              ctypes.c_void_p(mask.data_ptr()), mask.stride(1),
                                              mask.stride(2), _stream(dev)),
                  "esa_build_dense_mask")
        return mask.to(device)

    def layout(self, device: torch.device) -> ElasticLayout:
        """The block layout on ``device`` (built once, cached)."""
        device = torch.device(device)
        if device.index is None:
            device = torch.device(device.type, torch.cuda.current_device())
        lay = self._layouts.get(device)
        if lay is None:
            lay = ElasticLayout(self.pattern, device)
            self._layouts[device] = lay
        return lay

    def _get_prepared_indices_and_mask(self, kv_seq_len: int):
        """Rows ``[:kv_seq_len]`` of the cached index set (:574-590)."""
        if kv_seq_len > self.max_seq_len:
            raise ValueError(
                f"Input sequence length ({kv_seq_len}) exceeds the maximum length initialized "
                f"in the module ({self.max_seq_len}).")
        idx, msk = self.sparse_attention_indices, self.sparse_causal_mask
        if idx is None:
            # ("dense" registers no index buffers, as the reference's does not)
            idx, msk = self._create_elastic_sparse_indices(self.max_seq_len,
                                                           self._anchor.device)
        return idx[:, :kv_seq_len, :], msk[:, :kv_seq_len, :]

    @staticmethod
    def _positions(cache_position, q_len: int, kv_len: int, device: torch.device) -> torch.Tensor:
        """cache_position as int64 on ``device``.  Negative positions count
        from kv_len, as the reference's indexing of rows ``[:kv_len]`` counts
        them (:588, :602-608); the kernel applies that.  A host-side value is
        range-checked here (IndexError, as the reference's indexing raises); a
        device tensor is passed through unchecked, so a decode step never
        waits on the GPU: the kernel writes NaN for a row whose position is
        out of range."""
        if isinstance(cache_position, torch.Tensor) and cache_position.is_cuda:
            pos = cache_position.reshape(-1)
            if pos.dtype != torch.int64 or not pos.is_contiguous():
                pos = pos.to(torch.int64).contiguous()
            if pos.numel() != q_len:
                raise ValueError(f"cache_position has {pos.numel()} entries for {q_len} query "
                                 "rows")
            return pos if pos.device == device else pos.to(device)
        pos = torch.as_tensor(cache_position).to(torch.int64).reshape(-1)
        if pos.numel() != q_len:
            raise ValueError(f"cache_position has {pos.numel()} entries for {q_len} query rows")
        if bool(((pos < -kv_len) | (pos >= kv_len)).any()):
            raise IndexError(f"cache_position out of range for kv_len {kv_len}")
        return pos.to(device)

    def forward(self, query_states: torch.Tensor, key_states: torch.Tensor,
                value_states: torch.Tensor, cache_position: Optional[torch.LongTensor] = None
                ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        q, k, v = query_states, key_states, value_states
        _check_qkv(q, k, v)
        B, H, Lq, D = q.shape
        kv_len = k.shape[2]
        if kv_len > self.max_seq_len:                                     # :579-584
            raise ValueError(
                f"Input sequence length ({kv_len}) exceeds the maximum length initialized "
                f"in the module ({self.max_seq_len}).")
        if H != self.num_attention_heads or k.shape[1] != self.num_key_value_heads:
            raise ValueError(
                f"expected {self.num_attention_heads} query heads and "
                f"{self.num_key_value_heads} key/value heads; got {H} and {k.shape[1]}")
        pos = None
        if cache_position is None:
            if Lq > kv_len:
                raise ValueError(f"q_len ({Lq}) exceeds kv_len ({kv_len}) without cache_position")
        else:
            pos = self._positions(cache_position, Lq, kv_len, q.device)
        grad = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or
                                            v.requires_grad)
        # the naive path returns its attention weights (:680); it and the
        # dense path apply attention dropout in training mode (:674, :721),
        # the Triton path does not
        naive = self.implementation == "naive"
        dropout_p = (float(self.attention_dropout)
                     if self.training and self.implementation != "triton" else 0.0)
        band_ok = (q.dtype in MFMA_DTYPES and band_head_dim(D) and self.attention_length <= 64
                   and kv_len < (1 << 24))
        if pos is None and not naive and dropout_p == 0.0 and q.dtype in MFMA_DTYPES \
                and D not in (64, 128) and band_ok:
            # other head dims: the band forward on MFMA (zero padding up to 64,
            # 128 or 256), the gather backward
            if grad:
                o = _ElasticBandRowsAttention.apply(q, k, v, self.pattern, self.scaling, None)
                return o.reshape(B, Lq, H * D), None
            o, _ = elastic_attention_band(q, k, v, self.pattern, self.scaling, return_lse=False)
            return o.view(B, Lq, H * D), None                              # :761-763
        if pos is None and not naive and dropout_p == 0.0 and q.dtype in MFMA_DTYPES \
                and D in (64, 128):
            if grad:
                o = _ElasticTileAttention.apply(q, k, v, self.layout(q.device), self.scaling,
                                                self.prefill_kernel)
                return o.reshape(B, Lq, H * D), None
            o, _ = _prefill_fwd(q, k, v, self.layout(q.device), self.scaling, False, None, None,
                                None, self.prefill_kernel, True)
            return o.view(B, Lq, H * D), None                              # :761-763
        if pos is not None and not naive and dropout_p == 0.0 and band_ok \
                and Lq >= BAND_POSITION_MIN_ROWS \
                and (self.layer_idx == 0 or B * H * Lq * D > BAND_POSITION_MIN_UNITS * 128):
            # a chunked prefill: the band kernel at the given positions
            if grad:
                o = _ElasticBandRowsAttention.apply(q, k, v, self.pattern, self.scaling, pos)
                return o.reshape(B, Lq, H * D), None
            o, _ = elastic_attention_band(q, k, v, self.pattern, self.scaling, return_lse=False,
                                          positions=pos)
            return o.view(B, Lq, H * D), None                              # :761-763
        # per-row gather: decode rows, float32 / float16, other head dims, the
        # naive path; keep decisions of dropout drawn from torch's generator
        seed = int(torch.randint(0, 1 << 62, (1,)).item()) if dropout_p > 0.0 else 0
        if grad:
            o, wts = _ElasticRowsAttention.apply(q, k, v, self.pattern, self.scaling, pos,
                                                 dropout_p, seed, naive)
        else:
            got = _rows_fwd(q, k, v, self.pattern, self.scaling, pos, False, dropout_p, seed,
                            naive)
            o, wts = got[0], (got[2] if naive else None)
        return o.reshape(B, Lq, H * D), (wts if naive else None)          # :761-763
