"""Non-finite values in V (GPU).

The reference gathers only the K/V rows a query row attends
(elastic_sparse_attention.py:131-154), so an Inf or NaN in V row k reaches
exactly the rows that list k.  The per-row gather kernels (decode, float32,
the reference operator) keep that: rows that do not attend k are
bit-identical to a clean run.  The MFMA kernels stage whole key blocks or
bands and multiply p = 0 into the rows a query row does not attend, and
0 * Inf is NaN: a non-finite V row can also reach rows whose staged block
or band covers it without attending it.  That is a declared limitation
(the reference-exact test below is skipped); what holds for them is that
rows whose staged keys stay clear of k are bit-identical to a clean run.
"""
import pytest
import torch

from esa_oracle import elastic_indices, seeded_inputs
from elastic_sparse_attention import (ElasticLayout, elastic_attention_fwd,
                                      elastic_attention_rows, make_pattern)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def planted(B, H, L, D, dtype, key):
    q, k, v = seeded_inputs(B, H, H, L, D, dtype, seed=17, scale=1.0)
    vb = v.clone()
    vb[:, :, key, 3] = float("inf")
    return q, k, v, vb


def attends(idx, msk, key):
    """[H, L] bool: row i of head h lists `key` among its valid entries."""
    return ((idx == key) & msk.bool()).any(-1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_gather_path_reference_semantics(dtype):
    """The per-row gather: only rows attending the planted key change."""
    B, H, L, D, layer, key = 1, 4, 600, 64, 5, 300
    q, k, v, vb = planted(B, H, L, D, dtype, key)
    pat = make_pattern(L, 64, layer, 8, H)
    qd, kd = q.to(DEV), k.to(DEV)
    clean, _ = elastic_attention_rows(qd, kd, v.to(DEV), pat, D ** -0.5)
    bad, _ = elastic_attention_rows(qd, kd, vb.to(DEV), pat, D ** -0.5)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    hit = attends(idx, msk, key).T.unsqueeze(0).to(DEV)      # [1, L, H]
    assert bool(hit.any()) and bool((~hit).any())
    bad_f, clean_f = bad.float(), clean.float()
    assert bool((~torch.isfinite(bad_f[..., 3]))[hit.expand(B, L, H)].all())
    keep = (~hit).unsqueeze(-1).expand_as(bad_f)
    assert torch.equal(bad_f[keep], clean_f[keep])


@pytest.mark.parametrize("kernel,layer", [("band", 4), ("tile", 4), ("tile", 0)])
def test_mfma_paths_confine_nonfinite_v(kernel, layer):
    """The MFMA kernels: rows attending the planted key are non-finite, and
    rows whose staged keys (their 128-key neighbourhood of every listed key)
    stay clear of it are bit-identical to a clean run."""
    B, H, L, D, key = 1, 4, 2048, 128, 1000
    q, k, v, vb = planted(B, H, L, D, torch.bfloat16, key)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd = q.to(DEV), k.to(DEV)
    clean, _ = elastic_attention_fwd(qd, kd, v.to(DEV), lay, D ** -0.5, kernel=kernel)
    bad, _ = elastic_attention_fwd(qd, kd, vb.to(DEV), lay, D ** -0.5, kernel=kernel)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    hit = attends(idx, msk, key).T.unsqueeze(0).to(DEV)
    near = (((idx - key).abs() < 128) & msk.bool()).any(-1).T.unsqueeze(0).to(DEV)
    assert bool(hit.any())
    assert bool((~torch.isfinite(bad.float()[..., 3]))[hit].all())
    far = (~near).unsqueeze(-1).expand_as(bad)
    assert bool(far.any())
    assert torch.equal(bad[far], clean[far])


@pytest.mark.skip(reason="declared limitation: the MFMA kernels multiply p = 0 into staged V "
                         "rows a query row does not attend, so a non-finite value there reaches "
                         "that row; the per-row gather path keeps the reference's semantics")
@pytest.mark.parametrize("kernel,layer", [("band", 4), ("tile", 4), ("tile", 0)])
def test_mfma_paths_reference_semantics(kernel, layer):
    B, H, L, D, key = 1, 4, 2048, 128, 1000
    q, k, v, vb = planted(B, H, L, D, torch.bfloat16, key)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd = q.to(DEV), k.to(DEV)
    clean, _ = elastic_attention_fwd(qd, kd, v.to(DEV), lay, D ** -0.5, kernel=kernel)
    bad, _ = elastic_attention_fwd(qd, kd, vb.to(DEV), lay, D ** -0.5, kernel=kernel)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    hit = attends(idx, msk, key).T.unsqueeze(0).to(DEV)
    keep = (~hit).unsqueeze(-1).expand_as(bad)
    assert torch.equal(bad[keep], clean[keep])
