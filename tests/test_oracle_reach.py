"""The oracle's attention-hole reachability (check_attn_hole.py:53-180), pinned
by a computation that shares none of its steps, by closed forms and by the
reference's stated result.

Brute force: with A_l the boolean adjacency of layer l (A_l[i, j] = j is a
valid index of row i for some head, from ``dense_mask``), the reachable set
is r_last = e_p | A_last[p], then r <- r | (r A_l) for l = nl-2 .. 0, as
boolean matrix-vector products.
"""
import pytest
import torch

from esa_oracle import attention_reachability, dense_mask, elastic_indices


def brute_force(nl, H, w, pos):
    n = pos + 1
    r = torch.zeros(n, dtype=torch.bool)
    r[pos] = True
    counts = []
    for layer in range(nl - 1, -1, -1):
        idx, msk = elastic_indices(n, layer, nl, H, w)
        A = dense_mask(idx, msk).any(0).to(torch.float32)  # [n, n]
        if layer == nl - 1:
            r = r | A[pos].bool()
        else:
            r = r | ((r.to(torch.float32) @ A) > 0)
        counts.append(int(r.sum()))
    return r, counts


@pytest.mark.parametrize("nl,H,w,pos", [
    (8, 4, 8, 300), (8, 8, 16, 511), (3, 2, 5, 200), (12, 8, 32, 511),
    (2, 1, 4, 99), (5, 3, 6, 257), (8, 4, 64, 63), (4, 4, 16, 1),
])
def test_reachability_matches_dense_brute_force(nl, H, w, pos):
    r, c = attention_reachability(nl, H, w, pos)
    rb, cb = brute_force(nl, H, w, pos)
    assert torch.equal(r, rb)
    assert c == cb


def test_single_layer_is_the_sliding_window():
    # one layer: layer 0 is the window [p - w + 1, p]
    for w, pos in [(16, 100), (64, 1000), (7, 6), (5, 3)]:
        r, c = attention_reachability(1, 4, w, pos)
        want = torch.zeros(pos + 1, dtype=torch.bool)
        want[max(0, pos - w + 1):] = True
        assert torch.equal(r, want), (w, pos)
        assert c == [int(want.sum())]


def test_short_prefix_and_position_zero():
    # rows below w - 1 index their whole causal prefix at every layer
    for pos in (0, 1, 30, 62):
        r, c = attention_reachability(8, 8, 64, pos)
        assert bool(r.all()) and c == [pos + 1] * 8
    r, c = attention_reachability(5, 3, 16, 0)
    assert r.tolist() == [True] and c == [1] * 5


def test_counts_never_shrink_and_end_at_the_set_size():
    r, c = attention_reachability(8, 8, 16, 4095)
    assert all(a <= b for a, b in zip(c, c[1:]))
    assert c[-1] == int(r.sum())


@pytest.mark.slow
def test_reference_claim_no_holes_at_131072():
    # theory/note.md:85 and check_attn_hole.py:185-220: 8 layers, 8 heads,
    # w = 64 leave no hole at the last position
    r, c = attention_reachability(8, 8, 64, 131071)
    assert bool(r.all()) and c[-1] == 131072
