"""HIP forward kernels against the float32 oracle (GPU).

Bars (against an fp32 oracle on the same stored inputs): bf16 output
max-abs <= 2e-2, fp32 output max-abs <= 1e-4; lse is float32 natural log and
is held to 2e-3 (bf16) / 1e-4 (fp32).

At the full configured sizes the oracle runs on a seeded subset of query rows
(rows are independent, so this is exact for those rows), and every row is
covered by a size-independent cross-check: the block-sparse MFMA kernel
against the per-row gather kernel, two independent HIP paths.
"""
import pytest
import torch

from esa_oracle import (elastic_indices, forward_fp32, prepared_rows, scaling_for,
                        seeded_inputs)
from elastic_sparse_attention import (ElasticLayout, ElasticSparseAttention,
                                      ElasticSparseAttentionFunction, elastic_attention_band,
                                      elastic_attention_fwd, prefill_kernel, bwd_kernels,
                                      elastic_attention_rows, make_pattern,
                                      sparse_attention_fwd)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
BF16_TOL = 2e-2
BF16_LSE_TOL = 2e-3
F32_TOL = 1e-4


def oracle(q, k, v, idx, msk, sc, groups, rows=None):
    """fp32 oracle, optionally on a subset of query rows -> ([B,H,r,D], [B,H,r])."""
    if rows is not None:
        q = q[:, :, rows]
        idx = idx[:, rows]
        msk = msk[:, rows]
    return forward_fp32(q, k, v, idx, msk, sc, groups, chunk_rows=256)


def to_bhsd(o_bshd):
    return o_bshd.permute(0, 2, 1, 3)


def case(B, H, Hkv, L, D, dtype, layer, nl=8, w=64, seed=0, scale=None, outlier=0.0, Lq=None):
    scale = D ** -0.25 if scale is None else scale
    q, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=seed, scale=scale, outlier_frac=outlier,
                            Lq=Lq)
    idx, msk = elastic_indices(L, layer, nl, H, w)
    return q, k, v, idx, msk


# ---------------------------------------------------------------- block-sparse MFMA kernel
@pytest.mark.parametrize("D", [128, 64])
def test_tile_all_layers(D):
    B, H, L, w, nl = 1, 4, 1024, 64, 8
    for layer in range(nl):
        print(f"tile D={D} layer={layer}", flush=True)
        q, k, v, idx, msk = case(B, H, H, L, D, torch.bfloat16, layer, seed=layer)
        sc = scaling_for(D)
        lay = ElasticLayout(make_pattern(L, w, layer, nl, H), DEV)
        o, lse = elastic_attention_fwd(q.to(DEV), k.to(DEV), v.to(DEV), lay, sc, kernel="tile")
        ro, rl = oracle(q, k, v, idx, msk, sc, 1)
        assert (to_bhsd(o).float().cpu() - ro).abs().max().item() <= BF16_TOL
        assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


@pytest.mark.parametrize("B,H,Hkv,L,Lq,D,layer", [
    (2, 4, 2, 1000, 1000, 64, 3),     # GQA, partial last query block
    (1, 4, 4, 1024, 700, 128, 5),     # q_len < kv_len
    (3, 2, 1, 777, 777, 128, 6),      # batch, MQA, ragged length
    (1, 8, 8, 129, 129, 128, 2),      # one row past a block
    (1, 2, 2, 64, 64, 64, 7),         # shorter than one tile
])
def test_tile_shapes(B, H, Hkv, L, Lq, D, layer):
    print(f"tile shape B={B} H={H} Hkv={Hkv} L={L} Lq={Lq} D={D}", flush=True)
    q, k, v, idx, msk = case(B, H, Hkv, L, D, torch.bfloat16, layer, seed=11, Lq=Lq)
    sc = scaling_for(D)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    o, lse = elastic_attention_fwd(q.to(DEV), k.to(DEV), v.to(DEV), lay, sc, kernel="tile")
    pi, pm = prepared_rows(idx, msk, Lq, L, L)
    ro, rl = oracle(q, k, v, pi, pm, sc, H // Hkv)
    assert (to_bhsd(o).float().cpu() - ro).abs().max().item() <= BF16_TOL
    assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


@pytest.mark.parametrize("w", [32, 100, 128])
@pytest.mark.parametrize("D", [128, 64])
def test_tile_attention_lengths(w, D):
    """Index lists other than 64 entries: every bf16 prefill with
    attention_length > 64 runs the tile kernel (the band kernels take at most
    64), so it is checked at every layer, with GQA and a ragged q_len."""
    B, H, Hkv, L, Lq, nl = 2, 4, 2, 1100, 1037, 8
    for layer in range(nl):
        print(f"tile w={w} D={D} layer={layer}", flush=True)
        q, k, v, idx, msk = case(B, H, Hkv, L, D, torch.bfloat16, layer, w=w, seed=w + layer,
                                 scale=1.0, Lq=Lq)
        sc = scaling_for(D)
        lay = ElasticLayout(make_pattern(L, w, layer, nl, H), DEV)
        assert prefill_kernel(lay, Lq, B, D) == "tile" or w <= 64
        o, lse = elastic_attention_fwd(q.to(DEV), k.to(DEV), v.to(DEV), lay, sc, kernel="tile")
        pi, pm = prepared_rows(idx, msk, Lq, L, L)
        ro, rl = oracle(q, k, v, pi, pm, sc, H // Hkv)
        assert (to_bhsd(o).float().cpu() - ro).abs().max().item() <= BF16_TOL
        assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


def test_module_attention_length_128():
    """The drop-in module at attention_length = 128 (the tile kernel), bf16
    D = 128, against the oracle at every layer."""
    B, H, L, D, w = 1, 8, 2048, 128, 128
    for layer in (0, 2, 5, 7):
        m = ElasticSparseAttention(layer, 8, H, D, w, L)
        q, k, v, idx, msk = case(B, H, H, L, D, torch.bfloat16, layer, w=w, seed=layer)
        out, _ = m(q.to(DEV), k.to(DEV), v.to(DEV))
        ro, _ = oracle(q, k, v, idx, msk, m.scaling, 1)
        ref = ro.transpose(1, 2).reshape(B, L, H * D)
        assert (out.float().cpu() - ref).abs().max().item() <= BF16_TOL


def test_tile_unit_variance_logits():
    """N(0,1) inputs without the D^-0.25 scale (sharper softmax)."""
    q, k, v, idx, msk = case(1, 4, 4, 2048, 128, torch.bfloat16, 4, seed=5, scale=1.0)
    sc = scaling_for(128)
    lay = ElasticLayout(make_pattern(2048, 64, 4, 8, 4), DEV)
    o, lse = elastic_attention_fwd(q.to(DEV), k.to(DEV), v.to(DEV), lay, sc, kernel="tile")
    ro, rl = oracle(q, k, v, idx, msk, sc, 1)
    assert (to_bhsd(o).float().cpu() - ro).abs().max().item() <= BF16_TOL
    assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


def full_size_check(B, H, L, D, layer, scale, outlier, seed, n_rows=384, band=False):
    print(f"full size B={B} H={H} L={L} D={D} layer={layer} band={band}", flush=True)
    q, k, v = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=seed, scale=scale,
                            outlier_frac=outlier)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    sc = scaling_for(D)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    if band:
        o, lse = elastic_attention_band(qd, kd, vd, make_pattern(L, 64, layer, 8, H), sc)
    else:
        lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
        o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc, kernel="tile")
    g = torch.Generator().manual_seed(seed)
    rows = torch.cat([torch.tensor([0, 63, 64, 127, 128, L - 129, L - 1]),
                      torch.randint(0, L, (n_rows,), generator=g)]).unique()
    ro, rl = oracle(q, k, v, idx, msk, sc, 1, rows)
    oc = to_bhsd(o)[:, :, rows.to(DEV)].float().cpu()
    e_o = (oc - ro).abs().max().item()
    e_l = (lse[:, :, rows.to(DEV)].cpu() - rl).abs().max().item()
    print(f"  sampled rows vs oracle: o {e_o:.3e} lse {e_l:.3e}", flush=True)
    assert e_o <= BF16_TOL and e_l <= BF16_LSE_TOL
    # every row: against the per-row gather kernel run in float32 on the same
    # (bf16-valued) inputs, itself held to 1e-4 of the oracle
    # (test_rows_fp32_all_layers)
    og, lg = elastic_attention_rows(qd.float(), kd.float(), vd.float(),
                                    make_pattern(L, 64, layer, 8, H), sc)
    assert bool(torch.isfinite(o.float()).all())
    e_o = (o.float() - og).abs().max().item()
    e_l = (lse - lg).abs().max().item()
    print(f"  every row vs fp32 gather: o {e_o:.3e} lse {e_l:.3e}", flush=True)
    assert e_o <= BF16_TOL and e_l <= BF16_LSE_TOL


@pytest.mark.parametrize("bm,bn", [(64, 32), (128, 64), (128, 128)])
@pytest.mark.parametrize("L,H,layer,w", [(1000, 3, 5, 64), (777, 4, 7, 64), (513, 2, 2, 100),
                                         (300, 5, 1, 16)])
def test_stage_masks_match_oracle(bm, bn, L, H, layer, w):
    """esa_build_stage_masks: word q of stage st for row r holds exactly the
    row's valid keys (oracle index sets) among the stage's keys."""
    print(f"stage masks bm={bm} bn={bn} L={L} H={H} layer={layer} w={w}", flush=True)
    lay = ElasticLayout(make_pattern(L, w, layer, 8, H), DEV).stages(bn, bm)
    masks = lay.stage_masks()
    assert masks is not None
    nw = bn // 32
    got = masks.cpu()[:lay.num_tiles * bm * nw].view(lay.num_tiles, bm, nw).to(torch.int64)
    got = got & 0xFFFFFFFF
    idx, msk = elastic_indices(L, layer, 8, H, w)
    rp = lay.row_ptr_host.view(-1)
    ci = lay.col_idx[:lay.num_tiles].cpu().to(torch.int64)
    nqb = (L + bm - 1) // bm
    want = torch.zeros(lay.num_tiles, bm, nw, dtype=torch.int64)
    weights = (1 << torch.arange(32, dtype=torch.int64))
    for h in range(H):
        for qb in range(nqb):
            s0, s1 = int(rp[h * nqb + qb]), int(rp[h * nqb + qb + 1])
            if s0 == s1:
                continue
            rows = torch.arange(qb * bm, min((qb + 1) * bm, L))
            keys, ok = idx[h, rows], msk[h, rows].bool()               # [R, w]
            rel = keys.unsqueeze(0) - (ci[s0:s1] * bn).view(-1, 1, 1)   # [S, R, w]
            inr = ok.unsqueeze(0) & (rel >= 0) & (rel < bn)
            hit = torch.zeros(s1 - s0, len(rows), bn, dtype=torch.bool)
            si, ri, ei = torch.nonzero(inr, as_tuple=True)
            hit[si, ri, rel[si, ri, ei]] = True
            words = (hit.view(s1 - s0, len(rows), nw, 32).to(torch.int64) * weights).sum(-1)
            want[s0:s1, :len(rows)] = words
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,Hkv,L,Lq,D", [(2, 4, 2, 1000, 937, 64), (1, 8, 8, 2048, 2048, 128),
                                           (3, 2, 1, 777, 700, 128)])
def test_tile_stage_masks_bit_identical(dtype, B, H, Hkv, L, Lq, D):
    """The tile forward with per-stage masks loaded gives the same bits as
    with the in-kernel index walk, for both staging shapes and every
    dilated layer; and meets the oracle."""
    for layer in range(1, 8):
        print(f"tile masks {dtype} B={B} H={H} Hkv={Hkv} L={L} Lq={Lq} D={D} layer={layer}",
              flush=True)
        q, k, v, idx, msk = case(B, H, Hkv, L, D, dtype, layer, seed=layer + 5, Lq=Lq)
        qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
        lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
        sc = scaling_for(D)
        for qbk in ((64, 32), (128, 64)):
            assert lay.stages(qbk[1], qbk[0]).stage_masks() is not None
            o1, l1 = elastic_attention_fwd(qd, kd, vd, lay, sc, kernel="tile", query_block=qbk[0],
                                           key_block=qbk[1], stage_masks=True)
            o0, l0 = elastic_attention_fwd(qd, kd, vd, lay, sc, kernel="tile", query_block=qbk[0],
                                           key_block=qbk[1], stage_masks=False)
            assert torch.equal(o1, o0) and torch.equal(l1, l0)
        pi, pm = prepared_rows(idx, msk, Lq, L, L)
        ro, rl = oracle(q, k, v, pi, pm, sc, H // Hkv)
        assert (to_bhsd(o1).float().cpu() - ro).abs().max().item() <= BF16_TOL
        assert (l1.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


@pytest.mark.parametrize("B,H,Hkv,L,Lq,D,layer", [
    (1, 8, 8, 4096, 4096, 128, 4), (1, 8, 8, 4096, 4096, 128, 7), (1, 8, 8, 4096, 4096, 128, 0),
    (2, 8, 2, 3000, 2500, 64, 5), (1, 4, 4, 1000, 1000, 128, 1),
])
def test_stage_layout_matches_tile_layout(B, H, Hkv, L, Lq, D, layer):
    # 64-key stages (tile halves no row needs are skipped) against whole
    # 128-key tiles: the same blocks in the same order, so the same bits
    print(f"stages vs tiles B={B} H={H} Hkv={Hkv} L={L} Lq={Lq} D={D} layer={layer}", flush=True)
    q, k, v, _, _ = case(B, H, Hkv, L, D, torch.bfloat16, layer, seed=layer + 11, Lq=Lq)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    assert lay.stages(64, 128).num_tiles <= 2 * lay.num_tiles
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o64, l64 = elastic_attention_fwd(qd, kd, vd, lay, scaling_for(D), key_block=64,
                                     query_block=128, kernel="tile")
    o128, l128 = elastic_attention_fwd(qd, kd, vd, lay, scaling_for(D), key_block=128,
                                       query_block=128, kernel="tile")
    assert torch.equal(o64, o128) and torch.equal(l64, l128)
    # 64-row items of two waves over 32-key stages
    o32, l32 = elastic_attention_fwd(qd, kd, vd, lay, scaling_for(D), key_block=32,
                                     query_block=64, kernel="tile")
    assert torch.equal(o32, o128) and torch.equal(l32, l128)



@pytest.mark.parametrize("layer", [0, 4, 7])
def test_full_size_8k(layer):
    full_size_check(1, 32, 8192, 128, layer, 128 ** -0.25, 0.0, seed=20 + layer, n_rows=1024)


@pytest.mark.parametrize("layer", [0, 4, 7])
def test_full_size_headline_32k(layer):
    full_size_check(1, 32, 32768, 128, layer, 128 ** -0.25, 0.0, seed=30 + layer, n_rows=1024)


@pytest.mark.parametrize("layer", [0, 4, 7])
def test_full_size_batched_4k(layer):
    full_size_check(8, 16, 4096, 64, layer, 1.0, 0.0, seed=40 + layer, n_rows=1024)


@pytest.mark.parametrize("layer", [0, 4, 7])
def test_full_size_long_outliers_128k(layer):
    full_size_check(1, 8, 131072, 128, layer, 1.0, 0.01, seed=50 + layer, n_rows=512)


# ---------------------------------------------------------------- band-gathered kernel
@pytest.mark.parametrize("D", [128, 64])
def test_band_all_layers(D):
    B, H, L, w, nl = 1, 4, 1024, 64, 8
    for layer in range(nl):
        print(f"band D={D} layer={layer}", flush=True)
        q, k, v, idx, msk = case(B, H, H, L, D, torch.bfloat16, layer, seed=layer + 3)
        sc = scaling_for(D)
        o, lse = elastic_attention_band(q.to(DEV), k.to(DEV), v.to(DEV),
                                        make_pattern(L, w, layer, nl, H), sc)
        ro, rl = oracle(q, k, v, idx, msk, sc, 1)
        assert (to_bhsd(o).float().cpu() - ro).abs().max().item() <= BF16_TOL
        assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


@pytest.mark.parametrize("B,H,Hkv,L,Lq,D,layer,w,nl", [
    (2, 4, 2, 1000, 1000, 64, 3, 64, 8),    # GQA, partial last group
    (1, 4, 4, 1024, 700, 128, 5, 64, 8),    # q_len < kv_len
    (3, 2, 1, 777, 777, 128, 6, 64, 8),     # batch, MQA, ragged length
    (1, 2, 2, 17, 17, 128, 4, 64, 8),       # one row past a group
    (1, 2, 2, 5, 5, 64, 7, 64, 8),          # shorter than one group
    (1, 3, 3, 1024, 1024, 128, 1, 64, 8),   # odd head count: bands of 17 keys
    (1, 5, 5, 2048, 2048, 64, 4, 64, 8),    # odd head count, D = 64
    (1, 3, 3, 1024, 1024, 128, 4, 48, 6),   # w = 48, wide bands
    (1, 4, 4, 1024, 1024, 128, 2, 17, 4),   # w = 17
    (1, 1, 1, 1024, 1024, 128, 5, 32, 8),   # one head (t = 0)
    # entry spacing (q_len + 0) / w >= 1000 at the last layer: the kernel
    # that requests V after PV (the other refill order)
    (1, 3, 3, 16384, 16384, 64, 7, 16, 8),  # odd head count, D = 64
    (2, 2, 1, 12000, 12000, 128, 7, 12, 8),  # GQA, D = 128, spacing exactly 1000
    # interpolation weight 0: the sliding-window kernel
    (2, 4, 2, 1000, 1000, 64, 0, 64, 8),    # GQA, partial last group
    (1, 4, 4, 1024, 700, 128, 0, 64, 8),    # q_len < kv_len
    (1, 2, 2, 5, 5, 64, 0, 64, 8),          # shorter than one group
    (1, 3, 3, 1024, 1024, 128, 0, 48, 6),   # w = 48
    (1, 4, 4, 1024, 1024, 128, 0, 17, 4),   # w = 17: one chunk pair per group
    (3, 2, 1, 777, 777, 128, 0, 64, 1),     # one layer (weight 0), MQA, ragged length
    (1, 2, 2, 4096, 4096, 64, 0, 64, 8),    # many groups per XCD range
])
def test_band_shapes(B, H, Hkv, L, Lq, D, layer, w, nl):
    print(f"band shape B={B} H={H} Hkv={Hkv} L={L} Lq={Lq} D={D} layer={layer} w={w} nl={nl}",
          flush=True)
    q, k, v, idx, msk = case(B, H, Hkv, L, D, torch.bfloat16, layer, nl=nl, w=w, seed=13, Lq=Lq)
    sc = scaling_for(D)
    o, lse = elastic_attention_band(q.to(DEV), k.to(DEV), v.to(DEV),
                                    make_pattern(L, w, layer, nl, H), sc)
    pi, pm = prepared_rows(idx, msk, Lq, L, L)
    ro, rl = oracle(q, k, v, pi, pm, sc, H // Hkv)
    assert (to_bhsd(o).float().cpu() - ro).abs().max().item() <= BF16_TOL
    assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


def test_band_sharp_softmax_outliers():
    """N(0,1) inputs with x20 outlier channels: logits of std ~50 move the
    running max often (the rescale path)."""
    q, k, v, idx, msk = case(1, 4, 4, 2048, 128, torch.bfloat16, 4, seed=7, scale=1.0,
                             outlier=0.01)
    sc = scaling_for(128)
    o, lse = elastic_attention_band(q.to(DEV), k.to(DEV), v.to(DEV),
                                    make_pattern(2048, 64, 4, 8, 4), sc)
    ro, rl = oracle(q, k, v, idx, msk, sc, 1)
    assert (to_bhsd(o).float().cpu() - ro).abs().max().item() <= BF16_TOL
    assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


@pytest.mark.parametrize("L,H,B,D,layer,want,want_bwd", [
    (32768, 32, 1, 128, 4, "band", "band/band"), (32768, 32, 1, 128, 0, "band", "band/band"),
    (8192, 32, 1, 128, 3, "tile", "tile/tile"), (8192, 32, 1, 128, 4, "band", "band/band"),
    (4096, 32, 4, 128, 7, "tile", "tile/tile"),
    (8192, 32, 1, 128, 5, "band", "band/band"), (4096, 16, 8, 64, 6, "band", "band/tile"),
    (4096, 16, 8, 64, 7, "band", "band/tile"), (4096, 16, 8, 64, 4, "tile", "tile/tile"),
    (4096, 16, 8, 64, 5, "tile", "tile/tile"),
    (8192, 16, 4, 64, 3, "band", "band/tile"), (8192, 16, 4, 64, 4, "band", "band/band"),
    (16384, 16, 2, 64, 3, "band", "band/band"),
])
def test_prefill_kernel_choice(L, H, B, D, layer, want, want_bwd):
    # the measured crossovers: the band kernels where a group's rows stage
    # many 64 x 32 blocks, the tile kernels where they stage few (dQ and
    # dK/dV each at its own)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    assert prefill_kernel(lay, L, B, D) == want
    assert "/".join(bwd_kernels(lay, L, B, D)) == want_bwd


def test_band_rejects_unsupported():
    q = torch.zeros(1, 2, 64, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError):
        elastic_attention_band(q, q, q, make_pattern(64, 65, 3, 8, 2), 0.1)  # w > 64
    with pytest.raises(ValueError):
        elastic_attention_band(q.float(), q.float(), q.float(), make_pattern(64, 64, 3, 8, 2), 0.1)
    # head dims: multiples of 8 up to 256 (others padded up to 64, 128, 256)
    for bad_d in (100, 264):
        qd = torch.zeros(1, 2, 64, bad_d, dtype=torch.bfloat16, device=DEV)
        with pytest.raises(RuntimeError):
            elastic_attention_band(qd, qd, qd, make_pattern(64, 64, 3, 8, 2), 0.1)


@pytest.mark.parametrize("layer", [4, 7])
def test_band_full_size_headline_32k(layer):
    full_size_check(1, 32, 32768, 128, layer, 128 ** -0.25, 0.0, seed=60 + layer, n_rows=1024,
                    band=True)


def test_band_full_size_8k():
    full_size_check(1, 32, 8192, 128, 4, 128 ** -0.25, 0.0, seed=70, n_rows=1024, band=True)


def test_band_full_size_batched_4k():
    full_size_check(8, 16, 4096, 64, 7, 1.0, 0.0, seed=71, n_rows=1024, band=True)


def test_band_full_size_long_outliers_128k():
    full_size_check(1, 8, 131072, 128, 4, 1.0, 0.01, seed=72, n_rows=512, band=True)


# ---------------------------------------------------------------- per-row gather kernel
def test_rows_fp32_all_layers():
    """fp32 B=1 H=4 L=1024 D=64: output and lse within 1e-4 on every layer."""
    B, H, L, D, w, nl = 1, 4, 1024, 64, 64, 8
    for layer in range(nl):
        print(f"rows fp32 layer={layer}", flush=True)
        q, k, v, idx, msk = case(B, H, H, L, D, torch.float32, layer, seed=layer, scale=1.0)
        sc = scaling_for(D)
        o, lse = elastic_attention_rows(q.to(DEV), k.to(DEV), v.to(DEV),
                                        make_pattern(L, w, layer, nl, H), sc)
        ro, rl = oracle(q, k, v, idx, msk, sc, 1)
        assert (to_bhsd(o).cpu() - ro).abs().max().item() <= F32_TOL
        assert (lse.cpu() - rl).abs().max().item() <= F32_TOL


def test_rows_decode_positions():
    B, H, Hkv, L, D = 2, 8, 2, 3000, 128
    layer = 5
    _, k, v, idx, msk = case(B, H, Hkv, L, D, torch.bfloat16, layer, seed=3)
    q = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=4, scale=D ** -0.25, Lq=5)[0]
    pos = torch.tensor([0, 62, 1999, 2500, 2999])
    sc = scaling_for(D)
    o, lse = elastic_attention_rows(q.to(DEV), k.to(DEV), v.to(DEV),
                                    make_pattern(L, 64, layer, 8, H), sc, pos.to(DEV))
    pi, pm = prepared_rows(idx, msk, 5, L, L, pos)
    ro, rl = forward_fp32(q, k, v, pi, pm, sc, H // Hkv)
    assert (to_bhsd(o).float().cpu() - ro).abs().max().item() <= BF16_TOL
    assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


@pytest.mark.parametrize("dtype,D,w,layer", [
    (torch.float32, 128, 64, 4),    # 32-key chunks: two per row
    (torch.float32, 128, 100, 6),   # four chunks, the last partial
    (torch.bfloat16, 256, 64, 5),   # 32 lanes per row, 32-key chunks
    (torch.bfloat16, 128, 100, 7),  # 64-key chunks: two, the second partial
    (torch.float32, 256, 48, 2),    # 64 lanes per row, 16-key chunks
])
def test_rows_chunks_and_head_dims(dtype, D, w, layer):
    """The cooperative-row gather at every chunk split it uses (rows of D
    elements read by D * size / 16 lanes, chunks of 64 / 32 / 16 keys) and
    index lists longer than one chunk, against the float32 oracle."""
    B, H, Hkv, L = 1, 4, 2, 700
    print(f"rows {dtype} D={D} w={w} layer={layer}", flush=True)
    q, k, v, idx, msk = case(B, H, Hkv, L, D, dtype, layer, w=w, seed=w + D, scale=1.0)
    sc = scaling_for(D)
    o, lse = elastic_attention_rows(q.to(DEV), k.to(DEV), v.to(DEV),
                                    make_pattern(L, w, layer, 8, H), sc)
    ro, rl = oracle(q, k, v, idx, msk, sc, H // Hkv)
    tol, ltol = (F32_TOL, F32_TOL) if dtype == torch.float32 else (BF16_TOL, BF16_LSE_TOL)
    assert (to_bhsd(o).float().cpu() - ro).abs().max().item() <= tol
    assert (lse.cpu() - rl).abs().max().item() <= ltol


def test_rows_unaligned_rows_take_the_per_lane_gather():
    """bf16 K rows 132 elements apart (264 bytes: not a 16-byte multiple)
    take the per-lane gather; both kernels meet the bar against the oracle."""
    B, H, L, D, layer = 1, 2, 600, 128, 3
    q, k, v, idx, msk = case(B, H, H, L, D, torch.bfloat16, layer, seed=9, scale=1.0)
    kw = torch.zeros(B, H, L, 132, dtype=torch.bfloat16)
    kw[..., :D] = k
    sc = scaling_for(D)
    pat = make_pattern(L, 64, layer, 8, H)
    o1, l1 = elastic_attention_rows(q.to(DEV), kw.to(DEV)[..., :D], v.to(DEV), pat, sc)
    o2, l2 = elastic_attention_rows(q.to(DEV), k.to(DEV), v.to(DEV), pat, sc)
    ro, rl = oracle(q, k, v, idx, msk, sc, 1)
    for o, lse in ((o1, l1), (o2, l2)):
        assert (to_bhsd(o).float().cpu() - ro).abs().max().item() <= BF16_TOL
        assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


def test_operator_out_of_range_cooperative_rows():
    """Explicit indices with duplicates, out-of-range entries and an empty row
    at D = 128 (the cooperative-row gather): a valid out-of-range index scores
    0 against a zero key / value."""
    B, H, L, D, w = 1, 2, 300, 128, 80
    g = torch.Generator().manual_seed(5)
    q, k, v = seeded_inputs(B, H, H, L, D, torch.float32, seed=11)
    idx = torch.randint(-5, L + 5, (H, L, w), generator=g)
    idx[:, :, 3] = idx[:, :, 2]
    msk = (torch.rand(H, L, w, generator=g) > 0.2).long()
    msk[:, 11] = 0
    sc = 0.15
    o, lse = sparse_attention_fwd(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), msk.to(DEV), sc, 1)
    oor = (idx < 0) | (idx >= L)
    k2 = torch.cat([k, torch.zeros(B, H, 1, D)], dim=2)
    v2 = torch.cat([v, torch.zeros(B, H, 1, D)], dim=2)
    idx2 = torch.where(oor, torch.full_like(idx, L), idx)
    ro, rl = forward_fp32(q, k2, v2, idx2, msk, sc, 1)
    assert (o.cpu() - ro).abs().max().item() <= F32_TOL
    finite = torch.isfinite(rl)
    assert (lse.cpu()[finite] - rl[finite]).abs().max().item() <= F32_TOL
    assert torch.equal(o.cpu()[:, :, 11], torch.zeros(B, H, D))


# ---------------------------------------------------------------- explicit-index operator
@pytest.mark.parametrize("dtype,tol", [(torch.float32, F32_TOL), (torch.bfloat16, BF16_TOL)])
def test_operator_with_reference_indices(dtype, tol):
    B, H, Hkv, L, D, w = 2, 4, 2, 512, 64, 32
    q, k, v, idx, msk = case(B, H, Hkv, L, D, dtype, 6, w=w, seed=8, scale=1.0)
    sc = scaling_for(D)
    pi, pm = prepared_rows(idx, msk, L, L, L)
    o = ElasticSparseAttentionFunction.apply(q.to(DEV), k.to(DEV), v.to(DEV), pi.to(DEV),
                                             pm.to(DEV), sc, H // Hkv)
    ro, _ = oracle(q, k, v, pi, pm, sc, H // Hkv)
    assert o.shape == q.shape and o.dtype == dtype
    assert (o.float().cpu() - ro).abs().max().item() <= tol


def test_operator_arbitrary_indices_duplicates_out_of_range():
    """Duplicates count per entry; a valid out-of-range index scores 0 against
    a zero key/value, as the Triton gather mask does (:131-133)."""
    B, H, L, D, w = 1, 3, 200, 32, 24
    g = torch.Generator().manual_seed(2)
    q, k, v = seeded_inputs(B, H, H, L, D, torch.float32, seed=6)
    idx = torch.randint(-5, L + 5, (H, L, w), generator=g)
    idx[:, :, 1] = idx[:, :, 0]  # duplicates
    msk = (torch.rand(H, L, w, generator=g) > 0.3).long()
    msk[:, 7] = 0  # an empty row
    sc = 0.2
    o, lse = sparse_attention_fwd(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), msk.to(DEV), sc, 1)
    oor = (idx < 0) | (idx >= L)
    k2 = torch.cat([k, torch.zeros(B, H, 1, D)], dim=2)
    v2 = torch.cat([v, torch.zeros(B, H, 1, D)], dim=2)
    idx2 = torch.where(oor, torch.full_like(idx, L), idx)
    ro, rl = forward_fp32(q, k2, v2, idx2, msk, sc, 1)
    assert (o.cpu() - ro).abs().max().item() <= F32_TOL
    finite = torch.isfinite(rl)
    assert (lse.cpu()[finite] - rl[finite]).abs().max().item() <= F32_TOL
    assert torch.equal(o.cpu()[:, :, 7], torch.zeros(B, H, D))
    assert bool(torch.isinf(lse.cpu()[:, :, 7]).all())


# ---------------------------------------------------------------- the module, end to end
@pytest.mark.parametrize("dtype,D,tol", [(torch.bfloat16, 128, BF16_TOL),
                                         (torch.bfloat16, 64, BF16_TOL),
                                         (torch.float32, 64, F32_TOL)])
def test_module_forward_prefill(dtype, D, tol):
    B, H, Hkv, L = 2, 8, 4, 1024
    layer = 3
    m = ElasticSparseAttention(layer, 8, H, D, 64, 2048, num_key_value_heads=Hkv)
    q, k, v, idx, msk = case(B, H, Hkv, L, D, dtype, layer, seed=2, scale=1.0)
    out, wts = m(q.to(DEV), k.to(DEV), v.to(DEV))
    assert wts is None and out.shape == (B, L, H * D) and out.dtype == dtype
    ro, _ = oracle(q, k, v, idx, msk, m.scaling, m.num_kv_groups)
    ref = ro.transpose(1, 2).reshape(B, L, H * D)
    assert (out.float().cpu() - ref).abs().max().item() <= tol


def test_module_forward_decode_matches_prefill_rows():
    B, H, L, D = 1, 4, 600, 128
    m = ElasticSparseAttention(6, 8, H, D, 64, 1024)
    q, k, v, idx, msk = case(B, H, H, L, D, torch.bfloat16, 6, seed=9, scale=1.0)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    full, _ = m(qd, kd, vd)
    for pos in [0, 63, 599]:
        step, _ = m(qd[:, :, pos:pos + 1], kd[:, :, :pos + 1], vd[:, :, :pos + 1],
                    cache_position=torch.tensor([pos]))
        assert (step.float()[0, 0] - full.float()[0, pos]).abs().max().item() <= BF16_TOL
    with pytest.raises(IndexError):
        m(qd[:, :, :1], kd[:, :, :10], vd[:, :, :10], cache_position=torch.tensor([10]))
    with pytest.raises(ValueError, match="exceeds the maximum length"):
        big = torch.zeros(1, H, 1025, D, dtype=torch.bfloat16, device=DEV)
        m(big, big, big)


def test_module_decode_device_positions():
    """cache_position on the device goes to the kernel unchecked (no host
    synchronisation): negative positions count from kv_len as torch indexing
    does, and an out-of-range position gives a NaN row instead of an error;
    the other rows of the call are unaffected."""
    B, H, L, D = 2, 4, 300, 128
    m = ElasticSparseAttention(5, 8, H, D, 64, 512)
    q, k, v, idx, msk = case(B, H, H, L, D, torch.bfloat16, 5, seed=4, scale=1.0)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    full, _ = m(qd, kd, vd)
    rows = [7, 299, 150]
    got, _ = m(qd[:, :, rows], kd, vd, cache_position=torch.tensor([7, -1, -150], device=DEV))
    for n, r in enumerate(rows):
        assert (got.float()[:, n] - full.float()[:, r]).abs().max().item() <= BF16_TOL
    bad, _ = m(qd[:, :, [3, 4, 5]], kd, vd,
               cache_position=torch.tensor([3, 300, -301], device=DEV))
    assert (bad.float()[:, 0] - full.float()[:, 3]).abs().max().item() <= BF16_TOL
    assert bool(torch.isnan(bad.float()[:, 1:]).all())
    # the same positions from the host raise, as the reference's indexing does
    with pytest.raises(IndexError):
        m(qd[:, :, [3]], kd, vd, cache_position=torch.tensor([-301]))


def test_module_index_buffers_on_gpu():
    m = ElasticSparseAttention(2, 8, 4, 64, 64, 512)
    q = torch.zeros(1, 4, 8, 64, dtype=torch.bfloat16, device=DEV)
    m(q, q, q)
    ri, rm = elastic_indices(512, 2, 8, 4, 64)
    assert torch.equal(m.sparse_attention_indices.cpu(), ri)
    assert torch.equal(m.sparse_causal_mask.cpu(), rm)
    a, b = m._get_prepared_indices_and_mask(100)
    assert a.shape == (4, 100, 64)


@pytest.mark.parametrize("D", [64, 128])
def test_empty_inputs(D):
    """Batch 0 and zero query rows: empty outputs, nothing launched that
    could fault, through the module (prefill, decode, backward) and the
    kernels' own entry points."""
    H, L = 4, 256
    m = ElasticSparseAttention(3, 8, H, D, 64, L)
    for B, Lq, Lk in ((0, 256, 256), (0, 1, 256), (2, 0, 256)):
        print(f"empty B={B} Lq={Lq} Lk={Lk} D={D}", flush=True)
        q = torch.randn(B, H, Lq, D, device=DEV).bfloat16()
        k = torch.randn(B, H, Lk, D, device=DEV).bfloat16()
        v = torch.randn(B, H, Lk, D, device=DEV).bfloat16()
        lay = m.layout(DEV)
        for kern in ("tile", "band"):
            o, lse = elastic_attention_fwd(q, k, v, lay, m.scaling, kernel=kern)
            assert o.shape == (B, Lq, H, D) and lse.shape == (B, H, Lq)
        o, _ = elastic_attention_rows(q, k, v, lay.pattern, m.scaling, return_lse=False)
        assert o.shape == (B, Lq, H, D)
        if Lq == 1:
            cp = torch.full((1,), Lk - 1, device=DEV, dtype=torch.long)
            out, _ = m(q, k, v, cache_position=cp)
        else:
            out, _ = m(q, k, v)
        assert out.shape == (B, Lq, H * D)
        if Lq == Lk or Lq == 0:
            qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
            out, _ = m(qg, kg, vg)
            out.float().sum().backward()
            assert qg.grad.shape == q.shape and kg.grad.shape == k.shape
            assert vg.grad.shape == v.shape
            if kg.grad.numel():
                assert torch.count_nonzero(kg.grad) == 0 and torch.count_nonzero(vg.grad) == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("L,H,B,D,layer,split", [
    (4096, 16, 8, 64, 7, True), (8192, 32, 1, 128, 4, True), (4096, 16, 8, 64, 4, False),
    (1024, 4, 1, 128, 5, None),
])
def test_split_prefill(L, H, B, D, layer, split):
    """The module's row split (tile kernel on rows [0, R), band kernel at
    positions R .. on the rest): taken where the cost model puts it well
    below either kernel alone; its output and log-sum-exp agree with each
    kernel alone to bf16 rounding, and rows below R are the tile kernel's
    bits (the band kernel's rows start their entry walks at other entries
    than in a launch over all rows, so they agree to rounding)."""
    from elastic_sparse_attention import prefill_split
    print(f"split B={B} H={H} L={L} D={D} layer={layer}", flush=True)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    R = prefill_split(lay, L, B, D)
    if split is True:
        assert 0 < R < L and R % 128 == 0
    elif split is False:
        assert R in (0, L)
    q, k, v = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=layer, scale=1.0)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    sc = D ** -0.5
    o, lse = elastic_attention_fwd(q, k, v, lay, sc)
    ot, lt = elastic_attention_fwd(q, k, v, lay, sc, kernel="tile")
    ob, lb = elastic_attention_fwd(q, k, v, lay, sc, kernel="band")
    assert float((o.float() - ot.float()).abs().max()) <= 2e-2
    assert float((lse - lt).abs().max()) <= 2e-3
    assert float((o.float() - ob.float()).abs().max()) <= 2e-2
    assert float((lse - lb).abs().max()) <= 2e-3
    if 0 < R < L:
        assert torch.equal(o[:, :R], ot[:, :R]) and torch.equal(lse[..., :R], lt[..., :R])
