"""Non-finite values in K and V (GPU).

The reference gathers only the K/V rows a query row attends
(elastic_sparse_attention.py:131-154), so an Inf or NaN in K or V row k
reaches exactly the rows that list k.  The per-row gather kernels (decode,
float32, the reference operator) keep that bit for bit.  The MFMA prefill
kernels stage whole key blocks or bands: they mask scores by a select (so a
non-finite K value never reaches a row that does not list its key), and a
group or item whose output met a non-finite value runs again with the staged
V operands sanitised and the reference's non-finite values put back from the
row's own entries.  So for them too, rows that do not attend a planted key
are bit-identical to a clean run, and rows that do are non-finite exactly
where the per-row gather path is.  The MFMA backward flags every unit it
stores with a non-finite value and recomputes those on the reference's pairs,
so its gradients too are non-finite exactly where the per-row gather
backward's are.
"""
import pytest
import torch

from esa_oracle import elastic_indices, seeded_inputs
from elastic_sparse_attention import (ElasticLayout, elastic_attention_bwd,
                                      elastic_attention_bwd_rows, elastic_attention_fwd,
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


def rows_path(q, k, v, pat, D):
    o, _ = elastic_attention_rows(q, k, v, pat, D ** -0.5)
    return o


# (kernel, layer, L, H, D, w, dtype): the band kernel's early and late V
# refill orders (w = 2 at the last layer puts the entry spacing past 1000
# rows), both head dims, float16, its layer-0 (sliding-window) kernel, and
# the tile kernel's three staging shapes
NF_CASES = [("band", 4, 2048, 4, 128, 64, torch.bfloat16),
            ("band", 7, 2048, 4, 64, 64, torch.bfloat16),
            ("band", 7, 2048, 4, 128, 2, torch.bfloat16),
            ("band", 5, 1500, 3, 128, 64, torch.float16),
            ("band", 0, 2048, 4, 128, 64, torch.bfloat16),
            ("band", 0, 1500, 3, 64, 48, torch.float16),
            ("tile", 4, 2048, 4, 128, 64, torch.bfloat16),
            ("tile", 0, 2048, 4, 128, 64, torch.bfloat16),
            ("tile", 2, 1024, 4, 64, 64, torch.float16),
            ("tile64", 3, 1024, 4, 64, 64, torch.bfloat16),
            ("tile128", 6, 1024, 2, 128, 48, torch.bfloat16)]


def mfma(kernel, q, k, v, lay, D):
    if kernel == "tile64":
        o, _ = elastic_attention_fwd(q, k, v, lay, D ** -0.5, kernel="tile", query_block=64,
                                     key_block=32)
    elif kernel == "tile128":
        o, _ = elastic_attention_fwd(q, k, v, lay, D ** -0.5, kernel="tile", query_block=128,
                                     key_block=128)
    else:
        o, _ = elastic_attention_fwd(q, k, v, lay, D ** -0.5, kernel=kernel)
    return o


def same_nonfinite(a, b):
    """Same positions hold NaN, +Inf and -Inf in a and b."""
    a, b = a.float(), b.float()
    return (torch.equal(torch.isnan(a), torch.isnan(b)) and
            torch.equal(a == float("inf"), b == float("inf")) and
            torch.equal(a == float("-inf"), b == float("-inf")))


@pytest.mark.parametrize("kernel,layer,L,H,D,w,dtype", NF_CASES)
def test_mfma_paths_reference_semantics(kernel, layer, L, H, D, w, dtype):
    """V planted with +Inf, -Inf and NaN at three keys: every output row that
    attends none of them is bit-identical to a clean run of the same kernel,
    and the non-finite positions (and their kind) are those of the per-row
    gather path, which follows the reference's gather (:131-133, :152-154)."""
    print(f"nonfinite V {kernel} layer={layer} L={L} H={H} D={D} w={w} {dtype}", flush=True)
    q, k, v = seeded_inputs(1, H, H, L, D, dtype, seed=23, scale=1.0)
    keys = [L // 2 + 1, L // 3, L - 5]
    vb = v.clone()
    vb[:, :, keys[0], 3] = float("inf")
    vb[:, :, keys[1], D - 1] = float("nan")
    vb[:, :, keys[2], 7] = float("-inf")
    vb[:, :, keys[2], 8] = float("inf")
    pat = make_pattern(L, w, layer, 8, H)
    lay = ElasticLayout(pat, DEV)
    qd, kd = q.to(DEV), k.to(DEV)
    clean = mfma(kernel, qd, kd, v.to(DEV), lay, D)
    bad = mfma(kernel, qd, kd, vb.to(DEV), lay, D)
    ref = rows_path(qd, kd, vb.to(DEV), pat, D)
    idx, msk = elastic_indices(L, layer, 8, H, w)
    hit = torch.zeros(H, L, dtype=torch.bool)
    for key in keys:
        hit |= attends(idx, msk, key)
    hit = hit.T.unsqueeze(0).to(DEV)                                      # [1, L, H]
    assert bool(hit.any()) and bool((~hit).any())
    keep = (~hit).unsqueeze(-1).expand_as(bad)
    assert torch.equal(bad[keep], clean[keep])
    assert same_nonfinite(bad, ref)
    # the finite outputs of rows that attend a planted key agree with the
    # gather path to the bf16 bar (only the planted dims differ from clean)
    fin = torch.isfinite(ref.float()) & torch.isfinite(bad.float())
    assert float((bad.float() - ref.float())[fin].abs().max()) <= 2e-2


@pytest.mark.parametrize("kernel,layer,L,H,D,w,dtype", NF_CASES[:2] + NF_CASES[4:10])
def test_mfma_paths_nonfinite_k(kernel, layer, L, H, D, w, dtype):
    """K planted with +Inf, -Inf and NaN: a row attending a planted key gets a
    non-finite score there (NaN output, or, for a -Inf score, that key's
    probability is 0), exactly as the per-row gather path gives it; rows that
    attend no planted key are bit-identical to a clean run (the masked
    scores are selected away, never added to -inf)."""
    print(f"nonfinite K {kernel} layer={layer} L={L} H={H} D={D} w={w} {dtype}", flush=True)
    q, k, v = seeded_inputs(1, H, H, L, D, dtype, seed=29, scale=1.0)
    keys = [L // 2 + 3, L // 4, L - 9]
    kb = k.clone()
    kb[:, :, keys[0], 3] = float("inf")
    kb[:, :, keys[1], 5] = float("nan")
    kb[:, :, keys[2], 11] = float("-inf")
    pat = make_pattern(L, w, layer, 8, H)
    lay = ElasticLayout(pat, DEV)
    qd, vd = q.to(DEV), v.to(DEV)
    clean = mfma(kernel, qd, k.to(DEV), vd, lay, D)
    bad = mfma(kernel, qd, kb.to(DEV), vd, lay, D)
    ref = rows_path(qd, kb.to(DEV), vd, pat, D)
    idx, msk = elastic_indices(L, layer, 8, H, w)
    hit = torch.zeros(H, L, dtype=torch.bool)
    for key in keys:
        hit |= attends(idx, msk, key)
    hit = hit.T.unsqueeze(0).to(DEV)
    assert bool(hit.any()) and bool((~hit).any())
    keep = (~hit).unsqueeze(-1).expand_as(bad)
    assert torch.equal(bad[keep], clean[keep])
    assert same_nonfinite(bad, ref)
    fin = torch.isfinite(ref.float()) & torch.isfinite(bad.float())
    assert float((bad.float() - ref.float())[fin].abs().max()) <= 2e-2


# (dQ kernel / dK-dV kernel, layer, L, H, Hkv, D, dtype): each pair of the
# MFMA backward kernels, GQA, both head dims, float16, and the last layer's
# split of key block 0 over several waves (band dK/dV, groups * L > 6144)
BWD_NF_CASES = [("band/band", 4, 1024, 4, 2, 128, torch.bfloat16),
                ("tile/tile", 4, 1024, 4, 2, 128, torch.bfloat16),
                ("band/tile", 0, 1024, 4, 4, 64, torch.bfloat16),
                ("tile/band", 7, 1024, 4, 2, 64, torch.float16),
                ("tile/tile", 2, 700, 2, 1, 64, torch.float16),
                ("band/band", 7, 2048, 8, 2, 128, torch.bfloat16),
                ("band/band", 0, 1024, 4, 2, 128, torch.bfloat16),
                ("tile/band", 0, 700, 2, 1, 64, torch.float16)]


@pytest.mark.parametrize("where", ["v", "k"])
@pytest.mark.parametrize("kernels,layer,L,H,Hkv,D,dtype", BWD_NF_CASES)
def test_mfma_backward_reference_semantics(kernels, layer, L, H, Hkv, D, dtype, where):
    """V (or K) planted with +Inf, NaN and -Inf / +Inf at three keys, the
    forward output and log-sum-exp of the per-row gather (the reference's
    semantics): every gradient of the MFMA backward is non-finite exactly
    where the per-row gather backward's is, with the same kind (the kernels
    flag each 16-row dQ group and 16-key dK / dV block that met a non-finite
    value and bwd_fix_kernel recomputes those on the reference's pairs), and
    the finite values agree to the bf16 bar."""
    dq_kernel, dkdv_kernel = kernels.split("/")
    print(f"nonfinite bwd {where} {kernels} layer={layer} L={L} H={H} Hkv={Hkv} D={D} {dtype}",
          flush=True)
    q, k, v = seeded_inputs(1, H, Hkv, L, D, dtype, seed=31, scale=1.0)
    keys = [L // 2 + 1, L // 3, L - 5]
    t = (v if where == "v" else k).clone()
    t[:, :, keys[0], 3] = float("inf")
    t[:, :, keys[1], D - 1] = float("nan")
    t[:, :, keys[2], 7] = float("-inf")
    t[:, :, keys[2], 8] = float("inf")
    kb, vb = (k, t) if where == "v" else (t, v)
    pat = make_pattern(L, 64, layer, 8, H)
    lay = ElasticLayout(pat, DEV)
    qd, kd, vd = q.to(DEV), kb.to(DEV), vb.to(DEV)
    sc = D ** -0.5
    o, lse = elastic_attention_rows(qd, kd, vd, pat, sc)
    do = torch.randn(o.shape, generator=torch.Generator().manual_seed(5)).to(dtype).to(DEV)
    ref = elastic_attention_bwd_rows(qd, kd, vd, o, lse, do, pat, sc)
    got = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel=dq_kernel,
                                dkdv_kernel=dkdv_kernel)
    for name, g, r in zip(("dq", "dk", "dv"), got, ref):
        rf, gf = r.float(), g.float()
        fin = torch.isfinite(rf)
        print(f"  {name}: {int((~fin).sum())} non-finite of {rf.numel()}", flush=True)
        assert same_nonfinite(g, r), name
        assert bool(fin.any()), name
        err = float((gf - rf)[fin].abs().max())
        assert err <= 2e-2 * float(rf[fin].abs().max()), (name, err)
    # some gradient holds a non-finite value only because of the planted keys
    assert any(not bool(torch.isfinite(r.float()).all()) for r in ref)
