"""Pins the oracle's layout restatement (CPU only).

* golden SHA-256 hashes and sample rows written from the reference itself
  (tests/golden/make_golden.py imports elastic_sparse_attention.py and reads
  the buffers _create_elastic_sparse_indices fills, :470-535);
* an independent numpy float32 restatement, bit for bit;
* closed forms: layer 0 is a sliding window of width w, rows i < w - 1 are a
  dense causal prefix, the last layer's head 0 is rne(j * (i + 1) / w) and its
  last head ends on the diagonal;
* invariants: min(i + 1, w) valid entries per row, strictly rising, all
  <= i, masked entries 0, valid entries a prefix of j.
"""
import hashlib

import numpy as np
import pytest
import torch

from esa_oracle import block_layout, elastic_indices
from esa_oracle_np import elastic_indices_np


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().numpy().astype("<i8").tobytes()).hexdigest()


def test_golden_hashes(golden):
    """Every case the reference produced, hash for hash and row for row."""
    for c in golden["cases"]:
        if c["seq_len"] * c["heads"] > 8192 * 32:
            continue  # the full-size cases run in test_golden_hashes_full_size
        idx, msk = elastic_indices(c["seq_len"], c["layer_idx"], c["layers"], c["heads"], c["w"])
        assert sha(idx) == c["indices_sha256"], c
        assert sha(msk) == c["mask_sha256"], c
        assert int(msk.sum()) == c["valid_total"]
        for a, h in enumerate(c["sample_heads"]):
            for b, r in enumerate(c["sample_rows"]):
                assert idx[h, r].tolist() == c["indices_rows"][a][b]
                assert msk[h, r].tolist() == c["mask_rows"][a][b]


@pytest.mark.slow
def test_golden_hashes_full_size(golden):
    """The L = 32768 (H = 32) and L = 131072 (H = 8) cases."""
    n = 0
    for c in golden["cases"]:
        if c["seq_len"] * c["heads"] <= 8192 * 32:
            continue
        idx, msk = elastic_indices(c["seq_len"], c["layer_idx"], c["layers"], c["heads"], c["w"])
        assert sha(idx) == c["indices_sha256"], c
        assert sha(msk) == c["mask_sha256"], c
        n += 1
    assert n == 6


@pytest.mark.parametrize("L,H,w,nl", [(1024, 4, 64, 8), (700, 5, 48, 8), (900, 3, 100, 6),
                                      (333, 1, 16, 3), (257, 7, 33, 11), (64, 2, 64, 2)])
def test_numpy_restatement_agrees(L, H, w, nl):
    for layer in range(nl):
        a, b = elastic_indices(L, layer, nl, H, w)
        c, d = elastic_indices_np(L, layer, nl, H, w)
        np.testing.assert_array_equal(a.numpy(), c)
        np.testing.assert_array_equal(b.numpy(), d)


@pytest.mark.parametrize("w", [16, 64, 48])
def test_layer0_is_sliding_window(w):
    L, H = 600, 4
    idx, msk = elastic_indices(L, 0, 8, H, w)
    i = torch.arange(L).view(1, L, 1)
    j = torch.arange(w).view(1, 1, w)
    expect = torch.where(i >= w - 1, i - w + 1 + j, j)
    valid = (expect <= i)
    expect = torch.where(valid, expect, torch.zeros_like(expect))
    assert torch.equal(idx, expect.expand(H, L, w))
    assert torch.equal(msk, valid.long().expand(H, L, w))


@pytest.mark.parametrize("layer,nl", [(1, 8), (4, 8), (7, 8), (6, 12)])
def test_short_rows_are_dense_prefix(layer, nl):
    w, H = 64, 6
    idx, msk = elastic_indices(300, layer, nl, H, w)
    for i in range(w - 1):
        j = torch.arange(w)
        assert torch.equal(msk[:, i], (j <= i).long().expand(H, w))
        assert torch.equal(idx[:, i], torch.where(j <= i, j, 0).expand(H, w))


def test_last_layer_closed_form():
    L, H, w, nl = 2000, 5, 64, 8
    idx, msk = elastic_indices(L, nl - 1, nl, H, w)
    for i in [63, 64, 100, 1023, 1999]:
        sp = np.float32(i + 1) / np.float32(w)
        j = np.arange(w, dtype=np.float32)
        head0 = np.rint((j * sp).astype(np.float32)).astype(np.int64)
        assert idx[0, i].tolist() == head0.tolist()
        assert int(idx[H - 1, i, w - 1]) == i  # the last head ends on the diagonal


@pytest.mark.parametrize("L,H,w,nl", [(3000, 8, 64, 8), (2000, 6, 48, 5), (1500, 4, 100, 12)])
def test_invariants(L, H, w, nl):
    for layer in range(nl):
        idx, msk = elastic_indices(L, layer, nl, H, w)
        i = torch.arange(L).view(1, L, 1)
        cnt = msk.sum(-1)
        assert torch.equal(cnt, torch.clamp(torch.arange(L) + 1, max=w).expand(H, L))
        assert bool(((idx <= i) | (msk == 0)).all())
        assert bool((idx[msk == 0] == 0).all())
        # valid entries form a prefix of j and rise strictly
        assert bool((msk[..., 1:] <= msk[..., :-1]).all())
        d = idx[..., 1:] - idx[..., :-1]
        assert bool(((d > 0) | (msk[..., 1:] == 0)).all())


def test_block_layout_brute_force():
    L, H, w, nl = 1000, 3, 48, 6
    for layer in range(nl):
        idx, msk = elastic_indices(L, layer, nl, H, w)
        for bm, bn in [(128, 128), (64, 64), (128, 32)]:
            rp, ci = block_layout(idx, msk, bm, bn)
            nqb = (L + bm - 1) // bm
            for h in range(H):
                for qb in range(nqb):
                    rows = range(qb * bm, min(L, (qb + 1) * bm))
                    expect = sorted({int(idx[h, r, j]) // bn for r in rows for j in range(w)
                                     if msk[h, r, j]})
                    row = h * nqb + qb
                    got = ci[int(rp[row]):int(rp[row + 1])].tolist()
                    assert got == expect


@pytest.mark.slow
def test_headline_tile_counts():
    """Active 128 x 128 tiles at L = 32768, H = 32, w = 64, 8 layers."""
    expect = {0: 16352, 4: 563523, 7: 633512}
    for layer, n in expect.items():
        idx, msk = elastic_indices(32768, layer, 8, 32, 64)
        rp, _ = block_layout(idx, msk, 128, 128)
        assert int(rp[-1]) == n
