"""Pins the oracle's forward (CPU only).

forward_fp32 restates _naive_forward (elastic_sparse_attention.py:624-680)
in float32/float64 and adds the log-sum-exp the Triton kernel keeps as M and
L (:142-148, :165-166).  It is checked here against:
* brute-force dense masked softmax attention over the reference's full mask
  (_create_full_sparse_mask, :548-568), in float64;
* torch SDPA with a banded causal mask at layer 0, which is textbook
  sliding-window attention of width w;
* known answers: q = 0 gives uniform weights, so O is the mean of the valid
  V rows and lse = log(count) (the number of valid keys, min(i + 1, w));
* GQA through repeat_interleave equals MHA on repeated K/V (:632-634);
* the bf16 naive restatement (the CPU baseline) within the bf16 bound.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from esa_oracle import (dense_mask, elastic_indices, forward_fp32, naive_forward,
                        prepared_rows, scaling_for, seeded_inputs)


def brute_force(q, k, v, full, scaling, groups):
    kf = k.double().repeat_interleave(groups, dim=1)
    vf = v.double().repeat_interleave(groups, dim=1)
    s = torch.matmul(q.double(), kf.transpose(-1, -2)) * scaling
    s = s.masked_fill(~full.unsqueeze(0), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vf), lse


@pytest.mark.parametrize("layer,nl,w,H,groups", [(0, 8, 16, 4, 1), (3, 8, 16, 4, 2),
                                                 (7, 8, 16, 4, 4), (5, 12, 24, 6, 3)])
def test_forward_matches_dense_brute_force(layer, nl, w, H, groups):
    L, D, B = 160, 32, 2
    idx, msk = elastic_indices(L, layer, nl, H, w)
    q, k, v = seeded_inputs(B, H, H // groups, L, D, torch.float32, seed=layer + 10)
    sc = scaling_for(D)
    out, lse = forward_fp32(q, k, v, idx, msk, sc, groups, compute_dtype=torch.float64)
    ref, ref_lse = brute_force(q, k, v, dense_mask(idx, msk), sc, groups)
    torch.testing.assert_close(out, ref, rtol=0, atol=1e-12)
    torch.testing.assert_close(lse, ref_lse, rtol=0, atol=1e-12)


def test_layer0_equals_sliding_window_sdpa():
    L, D, H, w = 200, 64, 3, 32
    idx, msk = elastic_indices(L, 0, 8, H, w)
    q, k, v = seeded_inputs(1, H, H, L, D, torch.float32, seed=3)
    sc = scaling_for(D)
    out, _ = forward_fp32(q, k, v, idx, msk, sc, 1)
    i = torch.arange(L).view(L, 1)
    j = torch.arange(L).view(1, L)
    band = (j <= i) & (j > i - w)
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=band, scale=sc)
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("layer", [0, 2, 5])
def test_uniform_weights_known_answer(layer):
    L, D, H, w = 300, 16, 4, 20
    idx, msk = elastic_indices(L, layer, 6, H, w)
    _, k, v = seeded_inputs(1, H, H, L, D, torch.float32, seed=5)
    q = torch.zeros(1, H, L, D)
    out, lse = forward_fp32(q, k, v, idx, msk, 1.0, 1, compute_dtype=torch.float64)
    cnt = msk.sum(-1)
    assert torch.allclose(lse[0], torch.log(cnt.double()), atol=1e-12)
    for h in range(H):
        for i in [0, 5, 19, 20, 150, 299]:
            keys = idx[h, i][msk[h, i].bool()]
            assert torch.allclose(out[0, h, i], v[0, h, keys].double().mean(0), atol=1e-12)


def test_one_hot_scores_pick_one_key():
    """A key far above the rest takes all the weight: O = that V row."""
    L, D, H, w = 128, 8, 2, 16
    idx, msk = elastic_indices(L, 3, 8, H, w)
    k = torch.zeros(1, H, L, D)
    v = torch.randn(1, H, L, D, generator=torch.Generator().manual_seed(1))
    q = torch.zeros(1, H, L, D)
    i = 100
    target = int(idx[1, i, 5])
    k[0, 1, target, 0] = 1.0
    q[0, 1, i, 0] = 1000.0
    out, lse = forward_fp32(q, k, v, idx, msk, 1.0, 1, compute_dtype=torch.float64)
    assert torch.allclose(out[0, 1, i], v[0, 1, target].double(), atol=1e-9)
    assert abs(float(lse[0, 1, i]) - 1000.0) < 1e-9


def test_prepared_rows_slice_and_clamp():
    idx, msk = elastic_indices(512, 4, 8, 4, 32)
    a, b = prepared_rows(idx, msk, 100, 300, 512)
    assert a.shape == (4, 100, 32) and torch.equal(a, idx[:, :100])
    pos = torch.tensor([5, 299, 100])
    a, b = prepared_rows(idx, msk, 3, 300, 512, pos)
    assert torch.equal(a, idx[:, pos].clamp(0, 299)) and torch.equal(b, msk[:, pos])
    with pytest.raises(ValueError):
        prepared_rows(idx, msk, 10, 513, 512)


def test_naive_bf16_within_tolerance():
    """The reference fallback in bf16 (the CPU baseline) stays inside the
    bf16 bound of the float32 oracle on the same stored inputs."""
    L, D, H, w = 512, 128, 4, 64
    idx, msk = elastic_indices(L, 4, 8, H, w)
    q, k, v = seeded_inputs(1, H, H, L, D, torch.bfloat16, seed=7, scale=D ** -0.25)
    sc = scaling_for(D)
    ref, _ = forward_fp32(q, k, v, idx, msk, sc, 1)
    nv = naive_forward(q, k, v, idx, msk, sc, 1, L, chunk_rows=200)
    ref_flat = ref.transpose(1, 2).reshape(1, L, H * D)
    assert (nv.float() - ref_flat).abs().max().item() <= 2e-2


def test_naive_chunking_is_exact():
    L, D, H, w = 300, 32, 2, 16
    idx, msk = elastic_indices(L, 2, 4, H, w)
    q, k, v = seeded_inputs(2, H, H, L, D, torch.float32, seed=9)
    a = naive_forward(q, k, v, idx, msk, 0.3, 1, L)
    b = naive_forward(q, k, v, idx, msk, 0.3, 1, L, chunk_rows=37)
    assert torch.equal(a, b)


def test_naive_matches_fp32_oracle_in_fp32():
    L, D, H, w = 256, 64, 4, 32
    idx, msk = elastic_indices(L, 6, 8, H, w)
    q, k, v = seeded_inputs(1, H, 2, L, D, torch.float32, seed=11)
    sc = scaling_for(D)
    ref, _ = forward_fp32(q, k, v, idx, msk, sc, 2, compute_dtype=torch.float64)
    nv = naive_forward(q, k, v, idx, msk, sc, 2, L)
    assert (nv.double() - ref.transpose(1, 2).reshape(1, L, H * D)).abs().max() < 1e-5


def test_seeded_inputs_outliers():
    q, k, v = seeded_inputs(1, 2, 2, 64, 128, torch.float32, seed=1, outlier_frac=0.01)
    big_q = (q.abs().amax(dim=(0, 1, 2)) > 15).nonzero().view(-1)
    big_k = (k.abs().amax(dim=(0, 1, 2)) > 15).nonzero().view(-1)
    assert big_q.numel() == math.ceil(0.01 * 128) and torch.equal(big_q, big_k)
