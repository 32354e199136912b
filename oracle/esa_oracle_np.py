"""Second, independent restatement of the elastic layout in numpy float32.

TEST INFRASTRUCTURE ONLY (see esa_oracle.py).  Written row by row from the
formula the reference evaluates in ``elastic_sparse_attention.py:477-535``,
with every float32 operation rounded separately (numpy float32 arithmetic is
IEEE single with no contraction), ``np.rint`` for torch's round-half-to-even
and float32 true division.  Cross-checked bit for bit against
``esa_oracle.elastic_indices`` in the tests; the two share no code.
"""
from __future__ import annotations

import numpy as np

f32 = np.float32


def elastic_indices_np(seq_len: int, layer_idx: int, num_layers: int,
                       num_heads: int, w: int):
    """Returns ``(indices, mask)`` int64 ``[H, seq_len, w]`` like the torch
    restatement."""
    denom = num_layers - 1 if num_layers > 1 else 1
    alpha = layer_idx / denom                      # Python double
    a32 = f32(alpha)                               # scalar -> tensor dtype
    c32 = f32(w * (1 - alpha))                     # double product, then f32
    i = np.arange(seq_len, dtype=np.int64)
    end = np.maximum(w - 1, i)
    endp1 = (end + 1).astype(np.float32)
    pd = (c32 + (endp1 * a32).astype(f32)).astype(f32)
    st = np.rint((endp1 - pd).astype(f32)).astype(f32)
    st = np.maximum(st, f32(0)).astype(np.int64)
    win = end + 1 - st
    sp = (win.astype(f32) / f32(w)).astype(f32)
    j = np.arange(w + 1, dtype=np.int64).astype(f32)
    rel = np.rint((j[None, :] * sp[:, None]).astype(f32)).astype(np.int64)
    over = st[:, None] + rel
    base = over[:, :w].astype(f32)
    shifted = (over[:, 1:] - 1).astype(f32)
    if num_heads > 1:
        t = (np.arange(num_heads, dtype=np.int64).astype(f32) / f32(num_heads - 1)).astype(f32)
    else:
        t = np.zeros(1, dtype=f32)
    one_minus_t = (f32(1) - t).astype(f32)
    out = np.empty((num_heads, seq_len, w), dtype=np.int64)
    for h in range(num_heads):
        a = (base * one_minus_t[h]).astype(f32)
        b = (shifted * t[h]).astype(f32)
        out[h] = np.rint((a + b).astype(f32)).astype(np.int64)
    mask = out <= i[None, :, None]
    out[~mask] = 0
    return out, mask.astype(np.int64)
