"""Block-sparse MFMA backward against autograd through the float32 oracle (GPU).

The reference's ElasticSparseAttentionFunction.backward
(elastic_sparse_attention.py:299-339) returns dq, dk, dv of the forward; the
oracle's forward_fp32 restates that forward in differentiable torch ops, so
torch autograd through it (float32, on the bf16-valued inputs) is the
reference gradient.  bf16 bar: max |err| <= 2e-2 * max |ref| per tensor (P
and dS enter the MFMAs rounded to bf16, the gradients are stored in bf16).
The backward accumulates every gradient in one workgroup in a fixed order,
so two runs agree bit for bit.
"""
import pytest
import torch

from esa_oracle import elastic_indices, forward_fp32, prepared_rows, scaling_for, seeded_inputs
from elastic_sparse_attention import (ElasticLayout, ElasticSparseAttention, elastic_attention_bwd,
                                      elastic_attention_fwd, make_pattern)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
REL = 2e-2


def reference_grads(q, k, v, idx, msk, sc, groups, g):
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    o, _ = forward_fp32(qf, kf, vf, idx, msk, sc, groups, chunk_rows=512)
    (o * g).sum().backward()
    return qf.grad, kf.grad, vf.grad


def rel_err(got, ref, floor=1e-30):
    """max |got - ref| over max |ref|, the denominator at least `floor`."""
    return ((got.float().cpu() - ref).abs().max() / ref.abs().max().clamp_min(floor)).item()


@pytest.mark.parametrize("kernels", ["tile/tile", "band/tile", "band/band", "tile/band"])
@pytest.mark.parametrize("B,H,Hkv,L,Lq,D,layer", [
    (1, 4, 4, 1024, 1024, 128, 4),
    (1, 4, 4, 1024, 1024, 128, 0),
    (1, 4, 4, 1024, 1024, 128, 7),
    (1, 4, 4, 1024, 1024, 64, 3),
    (2, 8, 2, 640, 640, 128, 5),     # GQA, batch
    (1, 4, 4, 1000, 700, 128, 6),    # q_len < kv_len, ragged blocks
    (1, 2, 1, 200, 200, 64, 2),      # MQA, short
    (1, 3, 3, 1024, 1024, 128, 1),   # odd head count: bands of 17 keys (band dQ tail)
    (1, 6, 2, 777, 777, 64, 7),      # last layer: key 0 in every row of head 0
    (1, 2, 2, 64, 64, 128, 3),       # one row block, rows 0 .. w - 1 only
    (1, 8, 2, 2048, 2048, 128, 7),   # last layer, GQA: band dK/dV splits key block 0 (2 parts)
    (2, 4, 1, 3000, 3000, 64, 7),    # the same with batch 2, MQA, D = 64, ragged rows
    (2, 8, 2, 640, 640, 64, 0),      # layer 0 (a window): GQA, batch, D = 64
    (1, 4, 4, 1000, 700, 128, 0),    # layer 0, q_len < kv_len, ragged blocks
    (1, 2, 1, 40, 40, 128, 0),       # layer 0, fewer rows than the window
])
def test_backward_matches_autograd(B, H, Hkv, L, Lq, D, layer, kernels):
    """kernels: dQ kernel / dK-dV kernel."""
    dq_kernel, dkdv_kernel = kernels.split("/")
    print(f"bwd B={B} H={H} Hkv={Hkv} L={L} Lq={Lq} D={D} layer={layer} dq={dq_kernel} "
          f"dkdv={dkdv_kernel}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=layer + 3, scale=1.0, Lq=Lq)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    pi, pm = prepared_rows(idx, msk, Lq, L, L)
    sc = scaling_for(D)
    g = torch.randn(B, H, Lq, D, generator=torch.Generator().manual_seed(layer)).to(torch.bfloat16)
    rq, rk, rv = reference_grads(q, k, v, pi, pm, sc, H // Hkv, g.float())

    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc)
    do = g.to(DEV).permute(0, 2, 1, 3).contiguous()  # [B, Lq, H, D] like o
    dq, dk, dv = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel=dq_kernel,
                                       dkdv_kernel=dkdv_kernel)
    e = (rel_err(dq, rq), rel_err(dk, rk), rel_err(dv, rv))
    print(f"  rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert all(torch.isfinite(t.float()).all() for t in (dq, dk, dv))
    assert max(e) <= REL
    # deterministic: a second run is bit-identical
    dq2, dk2, dv2 = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel=dq_kernel,
                                          dkdv_kernel=dkdv_kernel)
    assert torch.equal(dq, dq2) and torch.equal(dk, dk2) and torch.equal(dv, dv2)


@pytest.mark.parametrize("kernels", ["tile/tile", "band/band"])
@pytest.mark.parametrize("B,H,Hkv,L,D,layer,w", [
    (1, 4, 2, 1000, 128, 5, 33),   # odd index-list length: lanes 33 .. 63 idle
    (1, 3, 1, 700, 64, 7, 16),     # short lists, last layer, MQA
    (2, 1, 1, 513, 128, 3, 64),    # one head (interpolation weight 0), ragged
    (1, 4, 2, 1000, 128, 0, 33),   # layer 0, odd window
    (1, 3, 1, 700, 64, 0, 16),     # layer 0, short window, MQA
    (1, 2, 1, 300, 128, 0, 1),     # layer 0, a window of one key (each row its own)
])
def test_backward_attention_lengths(B, H, Hkv, L, D, layer, w, kernels):
    """Index lists shorter than 64 entries and a single head, both halves of
    either kind, against autograd through the oracle.  Each error is taken
    relative to the larger of the tensor's own max |reference| and 1e-3 of
    the largest gradient: with a window of one key P = 1 exactly, so the
    reference dQ and dK are exactly zero and only rounding is left in the
    kernels' (dP - delta)."""
    dq_kernel, dkdv_kernel = kernels.split("/")
    print(f"bwd B={B} H={H} Hkv={Hkv} L={L} D={D} layer={layer} w={w} {kernels}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=layer + w, scale=1.0)
    idx, msk = elastic_indices(L, layer, 8, H, w)
    sc = scaling_for(D)
    g = torch.randn(B, H, L, D, generator=torch.Generator().manual_seed(w)).to(torch.bfloat16)
    rq, rk, rv = reference_grads(q, k, v, idx, msk, sc, H // Hkv, g.float())
    lay = ElasticLayout(make_pattern(L, w, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc)
    do = g.to(DEV).permute(0, 2, 1, 3).contiguous()
    dq, dk, dv = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel=dq_kernel,
                                       dkdv_kernel=dkdv_kernel)
    floor = 1e-3 * max(float(t.abs().max()) for t in (rq, rk, rv))
    e = (rel_err(dq, rq, floor), rel_err(dk, rk, floor), rel_err(dv, rv, floor))
    print(f"  rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert max(e) <= REL


@pytest.mark.parametrize("B,H,Hkv,L,Lq,D,w", [
    (1, 4, 4, 1024, 1024, 128, 64),
    (2, 8, 2, 1500, 1200, 64, 64),    # GQA, batch, q_len < kv_len, ragged blocks
    (1, 4, 2, 1100, 1100, 128, 100),  # longer index lists
])
def test_tile_dq_row_masks_bit_identical(B, H, Hkv, L, Lq, D, w):
    """The block-sparse dQ with the layout's row masks loaded gives the same
    bits as with the in-kernel index walk at every dilated layer (dK / dV
    untouched), and meets autograd at one of them."""
    for layer in range(1, 8):
        print(f"dq row masks B={B} H={H} Hkv={Hkv} L={L} Lq={Lq} D={D} w={w} layer={layer}",
              flush=True)
        q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=layer + 11, scale=1.0,
                                Lq=Lq)
        sc = scaling_for(D)
        lay = ElasticLayout(make_pattern(L, w, layer, 8, H), DEV)
        assert lay.stage_masks() is not None
        qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
        o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc, kernel="tile")
        g = torch.randn(B, H, Lq, D, generator=torch.Generator().manual_seed(layer))
        g = g.to(torch.bfloat16)
        do = g.to(DEV).permute(0, 2, 1, 3).contiguous()
        got = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel="tile",
                                    dkdv_kernel="tile", stage_masks=True)
        walk = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel="tile",
                                     dkdv_kernel="tile", stage_masks=False)
        assert all(torch.equal(x, y) for x, y in zip(got, walk))
        if layer == 5:
            idx, msk = elastic_indices(L, layer, 8, H, w)
            pi, pm = prepared_rows(idx, msk, Lq, L, L)
            ref = reference_grads(q, k, v, pi, pm, sc, H // Hkv, g.float())
            e = [rel_err(x, r) for x, r in zip(got, ref)]
            print(f"  rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
            assert max(e) <= REL


@pytest.mark.parametrize("B,H,Hkv,L,D,layer,w", [
    (1, 4, 2, 1100, 128, 4, 100),
    (1, 4, 4, 1024, 64, 6, 128),
    (2, 2, 1, 777, 128, 7, 128),
    (1, 4, 4, 1024, 128, 0, 128),
    (1, 4, 2, 900, 64, 2, 32),
])
def test_backward_tile_attention_lengths(B, H, Hkv, L, D, layer, w):
    """Index lists other than 64 entries through the block-sparse dQ and
    dK/dV (attention_length > 64 always takes them), against autograd."""
    print(f"bwd tile B={B} H={H} Hkv={Hkv} L={L} D={D} layer={layer} w={w}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=layer + w, scale=1.0)
    idx, msk = elastic_indices(L, layer, 8, H, w)
    sc = scaling_for(D)
    g = torch.randn(B, H, L, D, generator=torch.Generator().manual_seed(w)).to(torch.bfloat16)
    rq, rk, rv = reference_grads(q, k, v, idx, msk, sc, H // Hkv, g.float())
    lay = ElasticLayout(make_pattern(L, w, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc, kernel="tile")
    do = g.to(DEV).permute(0, 2, 1, 3).contiguous()
    dq, dk, dv = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel="tile",
                                       dkdv_kernel="tile")
    e = (rel_err(dq, rq), rel_err(dk, rk), rel_err(dv, rv))
    print(f"  rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert max(e) <= REL


def test_module_autograd_attention_length_128():
    """The module at attention_length = 128 backpropagates through the
    block-sparse kernels."""
    B, H, L, D, layer, w = 1, 4, 1024, 128, 5, 128
    m = ElasticSparseAttention(layer, 8, H, D, w, L)
    q, k, v = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=21, scale=1.0)
    idx, msk = elastic_indices(L, layer, 8, H, w)
    g = torch.randn(B, L, H * D, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out, _ = m(qd, kd, vd)
    (out.float() * g.to(DEV).float()).sum().backward()
    gref = g.float().view(B, L, H, D).permute(0, 2, 1, 3)
    rq, rk, rv = reference_grads(q, k, v, idx, msk, m.scaling, 1, gref)
    e = (rel_err(qd.grad, rq), rel_err(kd.grad, rk), rel_err(vd.grad, rv))
    print(f"  module w=128 rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert max(e) <= REL


def test_module_autograd():
    """The drop-in module's output backpropagates through the HIP backward."""
    B, H, L, D, layer = 1, 4, 768, 128, 4
    m = ElasticSparseAttention(layer, 8, H, D, 64, 1024)
    q, k, v = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=12, scale=1.0)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    g = torch.randn(B, L, H * D, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out, _ = m(qd, kd, vd)
    (out.float() * g.to(DEV).float()).sum().backward()
    gref = g.float().view(B, L, H, D).permute(0, 2, 1, 3)
    rq, rk, rv = reference_grads(q, k, v, idx, msk, m.scaling, 1, gref)
    e = (rel_err(qd.grad, rq), rel_err(kd.grad, rk), rel_err(vd.grad, rv))
    print(f"  module rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert max(e) <= REL


def test_backward_full_size_8k_layer4():
    """H = 32, L = 8192, D = 128 at layer 4: every gradient against autograd
    through the oracle on a 4-head slice (heads are independent)."""
    B, H, L, D, layer = 1, 32, 8192, 128, 4
    q, k, v = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=77, scale=128 ** -0.25)
    sc = scaling_for(D)
    g = torch.randn(B, H, L, D, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc)
    dq, dk, dv = elastic_attention_bwd(qd, kd, vd, o, lse, g.to(DEV).permute(0, 2, 1, 3).contiguous(),
                                       lay, sc)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    heads = [0, 13, 31]
    for h in heads:
        rq, rk, rv = reference_grads(q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1], idx[h:h + 1],
                                     msk[h:h + 1], sc, 1, g[:, h:h + 1].float())
        e = (rel_err(dq[:, h:h + 1], rq), rel_err(dk[:, h:h + 1], rk), rel_err(dv[:, h:h + 1], rv))
        print(f"  head {h} rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
        assert max(e) <= REL


def test_backward_last_layer_split_8k():
    """Last layer, GQA 8 / 2, L = 8192: the band dK/dV splits key block 0 of
    each kv head over 6 waves and adds their float32 partial sums in part
    order.  Each kv head's gradients against autograd through
    the oracle (the kv head's four query heads), and two runs bit-identical."""
    B, H, Hkv, L, D, layer = 1, 8, 2, 8192, 128, 7
    print(f"bwd last-layer split B={B} H={H} Hkv={Hkv} L={L} D={D}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=41, scale=D ** -0.25)
    sc = scaling_for(D)
    g = torch.randn(B, H, L, D, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc)
    do = g.to(DEV).permute(0, 2, 1, 3).contiguous()
    got = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel="band",
                                dkdv_kernel="band")
    again = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel="band",
                                  dkdv_kernel="band")
    assert all(torch.equal(x, y) for x, y in zip(got, again))
    dq, dk, dv = got
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    for kvh in range(Hkv):
        hs = slice(4 * kvh, 4 * kvh + 4)
        rq, rk, rv = reference_grads(q[:, hs], k[:, kvh:kvh + 1], v[:, kvh:kvh + 1], idx[hs],
                                     msk[hs], sc, 4, g[:, hs].float())
        e = (rel_err(dq[:, hs], rq), rel_err(dk[:, kvh:kvh + 1], rk),
             rel_err(dv[:, kvh:kvh + 1], rv))
        print(f"  kv head {kvh} rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
        assert max(e) <= REL


@pytest.mark.parametrize("kernels", ["tile/tile", "band/band"])
@pytest.mark.parametrize("B,H,Hkv,L,D,layer", [
    (1, 32, 32, 32768, 128, 4),   # the headline shape
    (1, 32, 32, 32768, 128, 7),   # last layer: band dK/dV splits key block 0 (6 parts)
    (1, 32, 8, 32768, 128, 7),    # GQA last layer (22 parts)
    (2, 8, 2, 8192, 64, 5),       # GQA, D = 64
    (1, 8, 8, 131072, 128, 4),    # the long-context configuration
])
def test_backward_identities_full_size(B, H, Hkv, L, D, layer, kernels):
    """Size-independent checks at full size.  Every row of P sums to one, so
    the sum of dV over a kv head's keys equals the sum of dO over the rows of
    its query heads; every row of dS = P (dP - delta) sums to zero, so the sum
    of dK over a kv head's keys is zero.  Both are compared against the sum
    of absolute values; without the identities the ratio would be about
    1 / sqrt(L) (random signs), here only rounding is left (P and dS enter
    the MFMAs in bf16, dK and dV are stored in bf16)."""
    dq_kernel, dkdv_kernel = kernels.split("/")
    print(f"bwd identities B={B} H={H} Hkv={Hkv} L={L} D={D} layer={layer} {kernels}",
          flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=90 + layer, scale=D ** -0.25)
    sc = scaling_for(D)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc)
    g = torch.Generator().manual_seed(layer)
    do = torch.randn(B, L, H, D, generator=g).to(torch.bfloat16).to(DEV)
    dq, dk, dv = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel=dq_kernel,
                                       dkdv_kernel=dkdv_kernel)
    assert all(bool(torch.isfinite(t.float()).all()) for t in (dq, dk, dv))
    groups = H // Hkv
    sum_do = do.float().sum(dim=1).view(B, Hkv, groups, D).sum(dim=2)      # [B, Hkv, D]
    sum_dv = dv.float().sum(dim=2)
    abs_dv = dv.float().abs().sum(dim=2)
    r_v = ((sum_dv - sum_do).abs() / abs_dv).max().item()
    r_k = (dk.float().sum(dim=2).abs() / dk.float().abs().sum(dim=2)).max().item()
    print(f"  |sum dV - sum dO| / sum|dV| {r_v:.3e}   |sum dK| / sum|dK| {r_k:.3e}   "
          f"(random signs: ~{L ** -0.5:.1e})", flush=True)
    # measured about 1e-4 at these shapes; a dropped delta term, a wrong lse
    # or a wrong scale gives ratios of order one
    assert r_v <= 1e-3 and r_k <= 1e-3


@pytest.mark.parametrize("B,H,Hkv,L,D,layer", [
    (1, 2, 2, 65536, 128, 4),
    (1, 4, 1, 32768, 128, 7),     # GQA, the last layer's split key block
    (1, 4, 4, 32768, 64, 5),
])
def test_few_heads_long_band_matches_tile(B, H, Hkv, L, D, layer):
    """Few heads at long lengths: grids of up to four rounds of resident
    waves whose heads' K / V (Q / dO) exceed an XCD's L2, where the band
    kernels walk every group or block from entry 0 instead of rotating.
    Forward O and LSE and all three gradients of the band kernels against
    the block-sparse kernels (independent paths), and a second band backward
    bit-identical."""
    print(f"few heads band vs tile B={B} H={H} Hkv={Hkv} L={L} D={D} layer={layer}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=130 + layer, scale=D ** -0.25)
    sc = scaling_for(D)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    ob, lb = elastic_attention_fwd(qd, kd, vd, lay, sc, kernel="band")
    ot, lt = elastic_attention_fwd(qd, kd, vd, lay, sc, kernel="tile")
    eo = (ob.float() - ot.float()).abs().max().item()
    el = (lb - lt).abs().max().item()
    print(f"  forward max|O band - O tile| {eo:.3e}  max|lse diff| {el:.3e}", flush=True)
    assert eo <= 2e-2 and el <= 2e-3
    do = torch.randn(B, L, H, D, generator=torch.Generator().manual_seed(layer))
    do = do.to(torch.bfloat16).to(DEV)
    tt = elastic_attention_bwd(qd, kd, vd, ot, lt, do, lay, sc, dq_kernel="tile",
                               dkdv_kernel="tile")
    bb = elastic_attention_bwd(qd, kd, vd, ot, lt, do, lay, sc, dq_kernel="band",
                               dkdv_kernel="band")
    for name, x, y in zip(("dq", "dk", "dv"), tt, bb):
        assert bool(torch.isfinite(y.float()).all())
        r = ((y.float() - x.float()).abs().max() / x.float().abs().max()).item()
        print(f"  max|{name} band - {name} tile| / max|{name}| {r:.3e}", flush=True)
        assert r <= REL
    again = elastic_attention_bwd(qd, kd, vd, ot, lt, do, lay, sc, dq_kernel="band",
                                  dkdv_kernel="band")
    assert all(torch.equal(x, y) for x, y in zip(bb, again))


@pytest.mark.parametrize("layer,Hkv", [(0, 32), (4, 32), (7, 32), (7, 8)])
def test_band_matches_tile_full_size(layer, Hkv):
    """The headline shape: dQ, dK and dV from the band kernels against the
    block-sparse kernels (independent paths over the same O and LSE), max
    |difference| <= 2e-2 * max |tile gradient| per tensor; each half of one
    kind leaves the other half bit-identical."""
    B, H, L, D = 1, 32, 32768, 128
    print(f"band vs tile backward B={B} H={H} Hkv={Hkv} L={L} D={D} layer={layer}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=110 + layer, scale=D ** -0.25)
    sc = scaling_for(D)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc)
    do = torch.randn(B, L, H, D, generator=torch.Generator().manual_seed(layer))
    do = do.to(torch.bfloat16).to(DEV)
    tt = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel="tile",
                               dkdv_kernel="tile")
    bt = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel="band",
                               dkdv_kernel="tile")
    bb = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel="band",
                               dkdv_kernel="band")
    for name, x, y in zip(("dq", "dk", "dv"), tt, bb):
        assert bool(torch.isfinite(y.float()).all())
        r = ((y.float() - x.float()).abs().max() / x.float().abs().max()).item()
        print(f"  max|{name} band - {name} tile| / max|{name}| {r:.3e}", flush=True)
        assert r <= REL
    assert torch.equal(tt[1], bt[1]) and torch.equal(tt[2], bt[2])
    assert torch.equal(bt[0], bb[0])


@pytest.mark.parametrize("kernels", ["tile/tile", "band/band"])
def test_strided_views_match_contiguous(kernels):
    """q, k, v as [B, H, L, D] views of [B, L, H, D] storage (a projection's
    output transposed, the usual caller layout): the forward and both
    backward halves read them through their strides, so O, LSE, dQ, dK and dV
    equal the contiguous inputs' bit for bit."""
    kind, dkdv_kind = kernels.split("/")
    B, H, Hkv, L, D, layer = 2, 8, 2, 1536, 128, 6
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=17, scale=D ** -0.25)
    sc = scaling_for(D)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qc, kc, vc = q.to(DEV), k.to(DEV), v.to(DEV)
    qs, ks, vs = (t.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for t in (q, k, v))
    assert not qs.is_contiguous() and torch.equal(qs, qc)
    g = torch.randn(B, L, H, D, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    do = g.to(DEV)
    res = []
    for qq, kk, vv in ((qc, kc, vc), (qs, ks, vs)):
        o, lse = elastic_attention_fwd(qq, kk, vv, lay, sc, kernel=kind)
        grads = elastic_attention_bwd(qq, kk, vv, o, lse, do, lay, sc, dq_kernel=kind,
                                      dkdv_kernel=dkdv_kind)
        res.append((o, lse) + tuple(grads))
    for name, x, y in zip(("o", "lse", "dq", "dk", "dv"), *res):
        assert torch.equal(x, y), name


@pytest.mark.parametrize("kernels", ["tile/tile", "band/tile", "band/band"])
def test_head_major_o_and_dout(kernels):
    """O and dO held head-major ([B, H, L, D] storage seen as [B, L, H, D])
    give the same gradients bit for bit as the forward's [B, L, H, D]
    layout: the delta pass (its own kernel beside a block-sparse half, the
    band dQ for the band pair) walks either layout in the same order."""
    dq_kind, dkdv_kind = kernels.split("/")
    B, H, Hkv, L, D, layer = 2, 8, 2, 1536, 128, 6
    print(f"head-major O/dO {kernels} B={B} H={H} Hkv={Hkv} L={L} D={D} layer={layer}",
          flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=19, scale=D ** -0.25)
    sc = scaling_for(D)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc)
    do = torch.randn(B, L, H, D, generator=torch.Generator().manual_seed(5))
    do = do.to(torch.bfloat16).to(DEV)
    ref = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel=dq_kind,
                                dkdv_kernel=dkdv_kind)
    oh, doh = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (o, do))
    assert oh.stride(2) > oh.stride(1) and torch.equal(oh, o) and torch.equal(doh, do)
    got = elastic_attention_bwd(qd, kd, vd, oh, lse, doh, lay, sc, dq_kernel=dq_kind,
                                dkdv_kernel=dkdv_kind)
    for name, x, y in zip(("dq", "dk", "dv"), ref, got):
        assert torch.equal(x, y), name


@pytest.mark.parametrize("D", [64, 128])
def test_band_dq_delta_matches_prep_kernel(D):
    """With both halves band the band dQ kernel forms delta = rowsum(dO * O)
    and lse2 itself; beside a block-sparse dK/dV they come from prep_kernel.
    Both sum each row in the same order, so the band dQ is the same bit for
    bit either way (GQA, a ragged q_len, the forward's [B, L, H, D] O)."""
    B, H, Hkv, L, Lq, layer = 2, 8, 2, 1300, 1237, 5
    print(f"band dQ delta vs prep_kernel D={D}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=23, scale=D ** -0.25, Lq=Lq)
    sc = scaling_for(D)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc)
    do = torch.randn(B, Lq, H, D, generator=torch.Generator().manual_seed(9))
    do = do.to(torch.bfloat16).to(DEV)
    own = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel="band",
                                dkdv_kernel="band")
    prep = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel="band",
                                 dkdv_kernel="tile")
    assert torch.equal(own[0], prep[0])
