"""CPU oracle for the elastic sparse attention forward.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this file:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or, for ``cpu_baseline``, as the
timed restatement of the reference's PyTorch fallback).  The HIP path never
routes through it.

It restates, with the same torch CPU ops, the reference's
``elastic_sparse_attention.py`` (HighCWu/elastic-sparse-attention):

* ``elastic_indices``       <- ``_create_elastic_sparse_indices`` (:470-535)
* ``prepared_rows``         <- ``_get_prepared_indices_and_mask`` (:574-590)
                               and the row slice / clamp of ``_triton_forward``
                               (:600-615)
* ``naive_forward``         <- ``_naive_forward`` (:624-680) with the one fix
                               the reference needs to run at all: it calls
                               ``_get_prepared_indices_and_mask(q_len, kv_len)``
                               (:638) but the method takes one argument (:574);
                               the restatement passes ``kv_len`` only.
* ``forward_fp32``          <- the same forward evaluated in float32 (or
                               float64) on inputs upcast from their stored
                               dtype, plus the log-sum-exp the Triton kernel
                               keeps as L and M (:142-148, :165-166).
* ``block_layout``          <- no reference code: the per-query-block set of
                               active KV tiles derived by brute-force set union
                               from ``elastic_indices``.
* ``dense_mask``            <- ``_create_full_sparse_mask`` (:537-572), used as
                               a brute-force cross-check at small sizes.
* ``attention_reachability`` <- ``check_attention_holes_pytorch`` in
                               ``check_attn_hole.py`` (:53-180): the tokens one
                               position reaches through all layers.

How each function is pinned (beyond restating the reference's ops):
  elastic_indices  golden SHA-256 hashes and slices written by importing the
                   reference (tests/golden/make_golden.py), an independent numpy
                   float32 restatement (esa_oracle_np.py), closed forms (layer 0
                   is a sliding window of width w; rows i < w-1 are dense causal
                   prefixes; the last layer's head 0 is rne(j*spacing)), and
                   invariants (min(i+1, w) distinct valid keys, all <= i).
  block_layout     brute-force per-row scan in the tests; invariants.
  forward_fp32     brute-force dense masked softmax attention on the
                   ``dense_mask`` at small L; torch SDPA with a banded mask at
                   layer 0 (textbook sliding-window attention); one-hot and
                   uniform-V known answers; the reference's dense path outputs
                   (golden fixtures).
  naive_forward    used only as the CPU baseline; its bf16 rounding points are
                   the reference's, checked against forward_fp32 within the
                   bf16 tolerance.
  attention_reachability  boolean products of the ``dense_mask`` adjacency
                   matrices at small sizes; closed forms (one layer = the
                   sliding window; a position below w reaches its whole
                   prefix; position 0 reaches only itself); the reference's
                   stated result (no holes at L = 131072, 8 layers, 8 heads,
                   w = 64, theory/note.md:85).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

__all__ = [
    "attention_reachability",
    "elastic_indices",
    "prepared_rows",
    "block_layout",
    "dense_mask",
    "forward_fp32",
    "naive_forward",
    "counted_tiles",
]


def elastic_indices(seq_len: int, layer_idx: int, num_hidden_layers: int,
                    num_attention_heads: int, attention_length: int
                    ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Elastic index set per (head, query position).

    Follows ``elastic_sparse_attention.py:477-535`` op for op on the CPU so
    that every float32 rounding (true division, separate multiply and add,
    round-half-to-even) happens exactly as in the reference.

    Returns ``(indices, mask)``, both int64 ``[H, seq_len, w]``; masked
    entries of ``indices`` are 0 (``:533``).
    """
    w = attention_length
    H = num_attention_heads
    dev = torch.device("cpu")
    current_ids = torch.arange(seq_len, device=dev)                       # :482
    end_ids = torch.max(torch.tensor(w, device=dev) - 1, current_ids)    # :483
    denominator = num_hidden_layers - 1 if num_hidden_layers > 1 else 1  # :488
    alpha = layer_idx / denominator                                      # :489
    ids_len = end_ids + 1                                                # :495
    position_distance = w * (1 - alpha) + ids_len * alpha                # :496
    start_ids_base = (end_ids + 1 - position_distance).round().clamp(min=0).long()  # :497
    window_lengths_base = end_ids + 1 - start_ids_base                   # :498
    spacing_base = window_lengths_base / w                               # :499
    steps_oversized = torch.arange(w + 1, device=dev)                    # :503
    rel = (steps_oversized[None, :] * spacing_base[:, None]).round().long()  # :505
    oversized = start_ids_base[:, None] + rel                            # :506
    base = oversized[:, :w]                                              # :510
    shifted = oversized[:, 1:] - 1                                       # :511
    heads = torch.arange(H, device=dev)                                  # :515
    interp = heads / (H - 1) if H > 1 else torch.zeros_like(heads)       # :516
    interp = interp.view(H, 1, 1)                                        # :520
    fidx = base.unsqueeze(0).float() * (1 - interp) + \
        shifted.unsqueeze(0).float() * interp                            # :521-522
    indices = fidx.round().long()                                        # :526
    mask = indices <= current_ids.view(1, -1, 1)                         # :532
    indices.masked_fill_(~mask, 0)                                       # :533
    return indices, mask.long()                                          # :535


def prepared_rows(indices: torch.Tensor, mask: torch.Tensor, q_len: int,
                  kv_len: int, max_seq_len: int,
                  cache_position: Optional[torch.Tensor] = None
                  ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Rows of the cached layout one forward uses.

    ``_get_prepared_indices_and_mask`` (:579-589) checks ``kv_len`` against
    ``max_seq_len`` and slices ``[:, :kv_len]``; ``_triton_forward`` then takes
    rows ``[:q_len]`` or ``[cache_position]`` (:602-611) and clamps to
    ``[0, kv_len - 1]`` (:615).
    """
    if kv_len > max_seq_len:
        raise ValueError(
            f"Input sequence length ({kv_len}) exceeds the maximum length "
            f"initialized in the module ({max_seq_len}).")
    idx = indices[:, :kv_len, :]
    msk = mask[:, :kv_len, :]
    if cache_position is not None:
        idx = idx[:, cache_position, :]
        msk = msk[:, cache_position, :]
    else:
        idx = idx[:, :q_len]
        msk = msk[:, :q_len]
    idx = torch.clamp(idx, min=0, max=kv_len - 1)
    return idx, msk


def block_layout(indices: torch.Tensor, mask: torch.Tensor, bm: int, bn: int
                 ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Active KV tiles per (head, query block) by brute-force set union.

    A tile ``kb`` is active for query block ``qb`` of head ``h`` when some row
    ``i`` in ``[qb*bm, (qb+1)*bm)`` has a valid entry with ``idx // bn == kb``.
    Returns ``row_ptr`` int32 ``[H * nqb + 1]`` (offsets into one flat
    ``col_idx``, rows ordered ``h * nqb + qb``) and ``col_idx`` int32, sorted
    ascending within each row.
    """
    H, L, w = indices.shape
    nqb = (L + bm - 1) // bm
    nkb = (L + bn - 1) // bn
    tiles = torch.div(indices, bn, rounding_mode="floor")
    qblock = torch.arange(L).div(bm, rounding_mode="floor").view(1, L, 1).expand(H, L, w)
    heads = torch.arange(H).view(H, 1, 1).expand(H, L, w)
    valid = mask.bool()
    flat = (heads[valid] * nqb + qblock[valid]) * nkb + tiles[valid]
    active = torch.zeros(H * nqb * nkb, dtype=torch.bool)
    active[flat] = True
    active = active.view(H, nqb, nkb)
    counts = active.sum(-1).to(torch.int32).view(-1)
    row_ptr = torch.zeros(H * nqb + 1, dtype=torch.int64)
    row_ptr[1:] = torch.cumsum(counts.to(torch.int64), 0)
    col_idx = torch.nonzero(active.view(H * nqb, nkb))[:, 1].to(torch.int32)
    return row_ptr.to(torch.int32), col_idx


def counted_tiles(row_ptr: torch.Tensor) -> int:
    """Number of active tiles in a layout (the metric's tile count)."""
    return int(row_ptr[-1])


def dense_mask(indices: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """Boolean ``[H, L, L]`` allowed-mask, as ``_create_full_sparse_mask``
    (:548-568) builds it: True at (h, i, idx) for every valid entry."""
    H, L, w = indices.shape
    full = torch.zeros(H, L, L, dtype=torch.bool)
    h_i = torch.arange(H).view(-1, 1, 1).expand_as(indices)
    q_i = torch.arange(L).view(1, -1, 1).expand_as(indices)
    k_i = indices.clamp(min=0, max=L - 1)
    valid = mask.bool()
    full[h_i[valid], q_i[valid], k_i[valid]] = True
    return full


def attention_reachability(num_hidden_layers: int, num_attention_heads: int,
                           attn_length: int, position: int):
    """Tokens ``position`` reaches through the layers, as
    ``check_attention_holes_pytorch`` (check_attn_hole.py:53-180) tracks them.

    The last layer starts the set with the position itself and its valid
    indices over all heads (:102-114); each earlier layer, from nl - 2 down to
    0, adds the valid indices of every token already in the set (:134-156).
    The reference stops once the set is the whole history (:161-163); a full
    set stays full, so running every layer gives the same final set.

    Returns ``(reach, counts)``: ``reach`` bool ``[position + 1]`` and the set
    size after each layer, last layer first.  A row's indices do not depend on
    the sequence length, so they come from ``elastic_indices`` over rows
    ``0..position``; the checker's own copy of the formula (:5-51) also
    requires idx >= 0 and leaves masked entries unfilled, which does not
    change the valid set.
    """
    n = position + 1
    reach = torch.zeros(n, dtype=torch.bool)
    reach[position] = True                                               # :114
    counts = []
    for layer in range(num_hidden_layers - 1, -1, -1):
        idx, msk = elastic_indices(n, layer, num_hidden_layers, num_attention_heads, attn_length)
        if layer == num_hidden_layers - 1:
            sources = torch.tensor([position])                           # :106-107
        else:
            sources = torch.where(reach)[0]                              # :141
        new = idx[:, sources, :][msk[:, sources, :].bool()].unique()     # :145-150
        new = new[new < n]                                               # :154
        reach[new] = True                                                # :156
        counts.append(int(reach.sum()))                                  # :158
        del idx, msk
    return reach, counts


def forward_fp32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 idx: torch.Tensor, msk: torch.Tensor, scaling: float,
                 num_kv_groups: int, compute_dtype: torch.dtype = torch.float32,
                 chunk_rows: int = 2048) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sparse attention forward evaluated in ``compute_dtype``.

    Inputs are upcast from their stored dtype.  ``idx``/``msk`` are the rows
    prepared by ``prepared_rows`` (``[H, Lq, w]``).  Semantics follow the
    reference's gather formulation (:655-678): for query row ``r`` of head
    ``h``, the output is ``sum_j softmax_j(scaling * q . k[idx_j]) v[idx_j]``
    over entries with ``msk == 1``; an entry listed twice counts twice.

    Returns ``(out [B, H, Lq, D], lse [B, H, Lq])``; ``lse`` is the natural
    log-sum-exp of the valid scaled scores, i.e. ``M + log(L)`` in the Triton
    kernel's terms (:142-148, :165-166).  Rows with no valid entry give output
    0 and lse ``-inf``.
    """
    B, H, Lq, D = q.shape
    qf = q.to(compute_dtype)
    kf = k.to(compute_dtype)
    vf = v.to(compute_dtype)
    if num_kv_groups > 1:                                                 # :632-634
        kf = kf.repeat_interleave(num_kv_groups, dim=1)
        vf = vf.repeat_interleave(num_kv_groups, dim=1)
    out = torch.empty(B, H, Lq, D, dtype=compute_dtype)
    lse = torch.empty(B, H, Lq, dtype=compute_dtype)
    neg_inf = float("-inf")
    for r0 in range(0, Lq, chunk_rows):
        r1 = min(Lq, r0 + chunk_rows)
        ci = idx[:, r0:r1]                                                # [H, c, w]
        cm = msk[:, r0:r1].bool()
        g = ci.unsqueeze(0).unsqueeze(-1).expand(B, -1, -1, -1, D)       # :655
        gk = torch.take_along_dim(kf.unsqueeze(2), g, dim=3)             # :659
        gv = torch.take_along_dim(vf.unsqueeze(2), g, dim=3)             # :660
        s = torch.matmul(qf[:, :, r0:r1].unsqueeze(3), gk.transpose(-1, -2)).squeeze(3)
        s = s * scaling                                                   # :664-665
        s = s.masked_fill(~cm.unsqueeze(0), neg_inf)                      # :669
        m = s.amax(dim=-1, keepdim=True)
        empty = torch.isinf(m) & (m < 0)
        m_safe = torch.where(empty, torch.zeros_like(m), m)
        p = torch.exp(s - m_safe)
        l = p.sum(dim=-1, keepdim=True)
        wgt = torch.where(empty, torch.zeros_like(p), p / torch.where(empty, torch.ones_like(l), l))
        out[:, :, r0:r1] = torch.matmul(wgt.unsqueeze(-2), gv).squeeze(-2)  # :678
        lse[:, :, r0:r1] = torch.where(empty, torch.full_like(m, neg_inf),
                                       m_safe + torch.log(l)).squeeze(-1)
    return out, lse


def naive_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  indices: torch.Tensor, mask: torch.Tensor, scaling: float,
                  num_kv_groups: int, max_seq_len: int,
                  cache_position: Optional[torch.Tensor] = None,
                  chunk_rows: Optional[int] = None) -> torch.Tensor:
    """The reference's PyTorch fallback, ``_naive_forward`` (:624-680), in the
    inputs' own dtype, with the :638 call fixed to ``(kv_len)``.

    ``indices``/``mask`` are the module's full cached buffers.  Rows are
    processed in chunks of ``chunk_rows`` query rows so the gathered
    ``[B, H, chunk, w, D]`` tensors stay bounded; rows are independent, so
    chunking leaves the result unchanged.  Returns the module output
    ``[B, Lq, H * D]`` (:761-763).  Dropout is 0 (inference).
    """
    B, H, Lq, D = q.shape
    kv_len = k.shape[2]
    if num_kv_groups > 1:                                                 # :632-634
        k = k.repeat_interleave(num_kv_groups, dim=1)
        v = v.repeat_interleave(num_kv_groups, dim=1)
    if kv_len > max_seq_len:                                              # :579-584
        raise ValueError(
            f"Input sequence length ({kv_len}) exceeds the maximum length "
            f"initialized in the module ({max_seq_len}).")
    ai = indices[:, :kv_len, :]                                           # :588
    am = mask[:, :kv_len, :]                                              # :589
    if cache_position is not None:                                        # :645-646
        ai = ai[:, cache_position, :]
        am = am[:, cache_position, :]
    else:                                                                 # :648-649
        ai = ai[:, :Lq]
        am = am[:, :Lq]
    out = torch.empty(B, H, Lq, D, dtype=q.dtype)
    step = Lq if chunk_rows is None else chunk_rows
    for r0 in range(0, Lq, step):
        r1 = min(Lq, r0 + step)
        ci = ai[:, r0:r1]
        cm = am[:, r0:r1]
        g = ci.unsqueeze(0).unsqueeze(-1).expand(B, -1, -1, -1, D)       # :655
        gk = torch.take_along_dim(k.unsqueeze(2), g, dim=3)             # :659
        gv = torch.take_along_dim(v.unsqueeze(2), g, dim=3)             # :660
        s = torch.matmul(q[:, :, r0:r1].unsqueeze(3), gk.transpose(-1, -2)).squeeze(3)  # :664
        s *= scaling                                                      # :665
        s.masked_fill_(cm.unsqueeze(0) < 1, torch.finfo(s.dtype).min)    # :669
        wgt = torch.softmax(s, dim=-1, dtype=torch.float32).type_as(q)    # :673
        out[:, :, r0:r1] = torch.matmul(wgt.unsqueeze(-2), gv).squeeze(-2)  # :678
    return out.transpose(1, 2).reshape(B, Lq, H * D)                      # :761-763


def scaling_for(head_dim: int) -> float:
    """``self.scaling = head_dim ** -0.5`` (:444)."""
    return head_dim ** -0.5


def seeded_inputs(B: int, H: int, Hkv: int, L: int, D: int, dtype: torch.dtype,
                  seed: int, scale: float = 1.0, outlier_frac: float = 0.0,
                  Lq: Optional[int] = None):
    """Synthetic q, k, v on the CPU: draw q, then k, then v in float32 from a
    seeded CPU generator, scale, optionally multiply ``ceil(frac*D)`` shared
    channels of q and k by 20, then cast to ``dtype``."""
    g = torch.Generator("cpu").manual_seed(seed)
    Lq = L if Lq is None else Lq
    q = torch.randn(B, H, Lq, D, generator=g) * scale
    k = torch.randn(B, Hkv, L, D, generator=g) * scale
    v = torch.randn(B, Hkv, L, D, generator=g)
    if outlier_frac > 0:
        n_out = int(math.ceil(outlier_frac * D))
        ch = torch.randperm(D, generator=g)[:n_out]
        q[..., ch] *= 20.0
        k[..., ch] *= 20.0
    if scale != 1.0:
        v = v * scale
    return q.to(dtype), k.to(dtype), v.to(dtype)
