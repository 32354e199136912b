"""Every forward kernel against the float32 oracle on seeded random shapes.

The fixed-case tests pick shapes by hand; this sweep draws them: head counts
with every GQA ratio, ragged lengths (q_len below kv_len, lengths that are
not multiples of any block), attention lengths from 8 to 100, 1 to 12
layers at any layer index, head dims 64 / 128 for the MFMA kernels and
others for the per-row gather, bf16 and fp16, flat and sharp logits.  Each
configuration runs the tile kernel at both staging shapes (with and without
stage masks), the band kernel where it applies (attention_length <= 64) and
the per-row gather, all against the oracle at the usual bars (bf16 / fp16
output 2e-2, lse 2e-3; float32 1e-4).  The backward sweep runs every
dQ / dK-dV kernel pair that applies against torch autograd through the
oracle (max error 2e-2 of the reference's max per gradient) and checks a
second run gives the same bits.
"""
import random

import pytest
import torch

from esa_oracle import elastic_indices, forward_fp32, prepared_rows, scaling_for, seeded_inputs
from elastic_sparse_attention import (ElasticLayout, elastic_attention_band, elastic_attention_bwd,
                                      elastic_attention_fwd, elastic_attention_rows, make_pattern)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TOL = {torch.bfloat16: (2e-2, 2e-3), torch.float16: (2e-2, 2e-3), torch.float32: (1e-4, 1e-4)}


def draw(seed):
    r = random.Random(seed)
    H = r.choice([1, 2, 3, 4, 6, 8])
    Hkv = r.choice([d for d in range(1, H + 1) if H % d == 0])
    L = r.randint(17, 1500)
    Lq = L if r.random() < 0.6 else r.randint(1, L)
    nl = r.choice([1, 2, 5, 8, 12])
    layer = r.randrange(nl)
    w = r.choice([8, 16, 24, 33, 48, 64, 64, 100])
    D = r.choice([64, 128, 128])
    dtype = r.choice([torch.bfloat16, torch.bfloat16, torch.float16])
    B = r.choice([1, 2])
    scale = r.choice([D ** -0.25, 1.0])
    return B, H, Hkv, L, Lq, D, nl, layer, w, dtype, scale


def check(o_bshd, lse, ro, rl, tol, ltol, what):
    got = o_bshd.permute(0, 2, 1, 3).float().cpu()
    err = (got - ro).abs().max().item()
    assert err <= tol, f"{what}: output max-abs {err:.3e} > {tol}"
    if lse is not None:
        lerr = (lse.cpu() - rl).abs().max().item()
        assert lerr <= ltol, f"{what}: lse max-abs {lerr:.3e} > {ltol}"


@pytest.mark.parametrize("seed", range(96))
def test_random_shapes_all_forward_kernels(seed):
    B, H, Hkv, L, Lq, D, nl, layer, w, dtype, scale = draw(seed)
    print(f"seed={seed} B={B} H={H} Hkv={Hkv} L={L} Lq={Lq} D={D} nl={nl} layer={layer} w={w} "
          f"{dtype} scale={scale:.3f}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=100 + seed, scale=scale, Lq=Lq)
    idx, msk = elastic_indices(L, layer, nl, H, w)
    pi, pm = prepared_rows(idx, msk, Lq, L, L)
    sc = scaling_for(D)
    ro, rl = forward_fp32(q, k, v, pi, pm, sc, H // Hkv)
    tol, ltol = TOL[dtype]
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    lay = ElasticLayout(make_pattern(L, w, layer, nl, H), DEV)
    for qb, kb in ((128, 64), (64, 32), (128, 128)):
        for masks in (True, False):
            o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc, kernel="tile", query_block=qb,
                                           key_block=kb, stage_masks=masks)
            check(o, lse, ro, rl, tol, ltol, f"tile {qb}x{kb} masks={masks}")
    if w <= 64:
        o, lse = elastic_attention_band(qd, kd, vd, lay.pattern, sc)
        check(o, lse, ro, rl, tol, ltol, "band")
    o, lse = elastic_attention_rows(qd, kd, vd, lay.pattern, sc)
    check(o, lse, ro, rl, tol, ltol, "rows")


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_rows_float32_any_head_dim(seed):
    """The per-row gather in float32 at head dims the MFMA kernels do not
    take (multiples of 4 up to 256)."""
    r = random.Random(1000 + seed)
    H = r.choice([1, 2, 4, 8])
    Hkv = r.choice([d for d in range(1, H + 1) if H % d == 0])
    L = r.randint(5, 900)
    Lq = L if r.random() < 0.5 else r.randint(1, L)
    nl = r.choice([1, 4, 8])
    layer = r.randrange(nl)
    w = r.choice([8, 32, 64, 100])
    D = r.choice([4, 32, 60, 96, 160, 256])
    B = r.choice([1, 3])
    print(f"rows fp32 seed={seed} B={B} H={H} Hkv={Hkv} L={L} Lq={Lq} D={D} nl={nl} "
          f"layer={layer} w={w}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.float32, seed=200 + seed, Lq=Lq)
    idx, msk = elastic_indices(L, layer, nl, H, w)
    pi, pm = prepared_rows(idx, msk, Lq, L, L)
    sc = scaling_for(D)
    ro, rl = forward_fp32(q, k, v, pi, pm, sc, H // Hkv)
    lay_pattern = make_pattern(L, w, layer, nl, H)
    o, lse = elastic_attention_rows(q.to(DEV), k.to(DEV), v.to(DEV), lay_pattern, sc)
    check(o, lse, ro, rl, 1e-4, 1e-4, "rows fp32")


def rel_err(got, ref):
    return ((got.float().cpu() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_backward(seed):
    B, H, Hkv, L, Lq, D, nl, layer, w, dtype, scale = draw(500 + seed)
    print(f"bwd seed={seed} B={B} H={H} Hkv={Hkv} L={L} Lq={Lq} D={D} nl={nl} layer={layer} "
          f"w={w} {dtype} scale={scale:.3f}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=300 + seed, scale=scale, Lq=Lq)
    idx, msk = elastic_indices(L, layer, nl, H, w)
    pi, pm = prepared_rows(idx, msk, Lq, L, L)
    sc = scaling_for(D)
    g = torch.randn(B, H, Lq, D, generator=torch.Generator().manual_seed(seed)).to(dtype)
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    ro, _ = forward_fp32(qf, kf, vf, pi, pm, sc, H // Hkv, chunk_rows=512)
    (ro * g.float()).sum().backward()
    refs = (qf.grad, kf.grad, vf.grad)
    lay = ElasticLayout(make_pattern(L, w, layer, nl, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc, kernel="tile")
    do = g.to(DEV).permute(0, 2, 1, 3).contiguous()
    pairs = [("tile", "tile")]
    if w <= 64:
        pairs += [("band", "band"), ("band", "tile"), ("tile", "band")]
    for dqk, dkvk in pairs:
        got = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel=dqk,
                                    dkdv_kernel=dkvk)
        errs = [rel_err(x, r) for x, r in zip(got, refs)]
        print(f"  {dqk}/{dkvk} rel err dq {errs[0]:.2e} dk {errs[1]:.2e} dv {errs[2]:.2e}",
              flush=True)
        assert max(errs) <= 2e-2, (dqk, dkvk, errs)
        again = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel=dqk,
                                      dkdv_kernel=dkvk)
        assert all(torch.equal(x, y) for x, y in zip(got, again))


@pytest.mark.parametrize("seed", range(16))
def test_random_decode_positions_through_module(seed):
    """The module's cache_position branch (the per-row gather) at random
    positions, negative ones included, with GQA, bf16 / fp16 / float32 and
    any head dim the gather takes, against the oracle's rows at those
    positions."""
    from elastic_sparse_attention import ElasticSparseAttention
    r = random.Random(2000 + seed)
    H = r.choice([2, 4, 8])
    Hkv = r.choice([d for d in range(1, H + 1) if H % d == 0])
    L = r.randint(40, 1200)
    max_len = L + r.choice([0, 17, 300])
    nq = r.choice([1, 1, 3, 8])
    nl = r.choice([2, 8, 12])
    layer = r.randrange(nl)
    w = r.choice([16, 64, 100])
    D = r.choice([64, 128, 96])
    dtype = r.choice([torch.bfloat16, torch.float16, torch.float32])
    B = r.choice([1, 4])
    pos = torch.tensor([r.randrange(-L, L) for _ in range(nq)], dtype=torch.int64)
    print(f"decode seed={seed} B={B} H={H} Hkv={Hkv} L={L} max={max_len} rows={nq} D={D} "
          f"nl={nl} layer={layer} w={w} {dtype} pos={pos.tolist()}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=400 + seed, scale=D ** -0.25, Lq=nq)
    idx, msk = elastic_indices(max_len, layer, nl, H, w)
    pi, pm = prepared_rows(idx, msk, nq, L, max_len, cache_position=pos)
    m = ElasticSparseAttention(layer, nl, H, D, w, max_len, num_key_value_heads=Hkv)
    ro, _ = forward_fp32(q, k, v, pi, pm, m.scaling, H // Hkv)
    out, _ = m(q.to(DEV), k.to(DEV), v.to(DEV), cache_position=pos.to(DEV))
    ref = ro.transpose(1, 2).reshape(B, nq, H * D)
    tol = TOL[dtype][0]
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= tol, err


def draw_chunk(seed):
    r = random.Random(3000 + seed)
    H = r.choice([2, 4, 8])
    Hkv = r.choice([d for d in range(1, H + 1) if H % d == 0])
    L = r.randint(200, 2000)
    nq = r.randint(32, min(600, L))
    p0 = r.randint(0, L - nq)
    nl = r.choice([1, 2, 8, 12])
    layer = r.randrange(nl)
    w = r.choice([16, 33, 64, 64])
    D = r.choice([64, 128, 128, 96])
    dtype = r.choice([torch.bfloat16, torch.bfloat16, torch.float16])
    B = r.choice([1, 2])
    pos = torch.arange(p0, p0 + nq, dtype=torch.int64)
    if r.random() < 0.25:  # a few rows moved or given as negatives: those groups take the gather
        for _ in range(r.randint(1, 3)):
            j = r.randrange(nq)
            pos[j] = r.randrange(-L, L)
    return B, H, Hkv, L, nq, nl, layer, w, D, dtype, pos


@pytest.mark.parametrize("seed", range(16))
def test_random_chunk_positions_through_module(seed):
    """The module's cache_position branch with a chunk of 32 or more rows (a
    chunked prefill: the band kernel, or the window kernel at layer 0, at the
    rows' positions; groups whose positions are not consecutive take the
    per-row gather) at random offsets, lengths, layers, GQA, bf16 / fp16 and
    head dims 64 / 96 / 128, against the oracle's rows at those positions."""
    from elastic_sparse_attention import ElasticSparseAttention
    B, H, Hkv, L, nq, nl, layer, w, D, dtype, pos = draw_chunk(seed)
    print(f"chunk seed={seed} B={B} H={H} Hkv={Hkv} L={L} rows={nq} p0={int(pos[0])} D={D} "
          f"nl={nl} layer={layer} w={w} {dtype}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=500 + seed, scale=D ** -0.25, Lq=nq)
    idx, msk = elastic_indices(L, layer, nl, H, w)
    pi, pm = prepared_rows(idx, msk, nq, L, L, cache_position=pos)
    m = ElasticSparseAttention(layer, nl, H, D, w, L, num_key_value_heads=Hkv)
    ro, _ = forward_fp32(q, k, v, pi, pm, m.scaling, H // Hkv)
    out, _ = m(q.to(DEV), k.to(DEV), v.to(DEV), cache_position=pos.to(DEV))
    ref = ro.transpose(1, 2).reshape(B, nq, H * D)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= TOL[dtype][0], err


@pytest.mark.parametrize("seed", range(16))
def test_random_strided_inputs_same_bits(seed):
    """q, k, v as the [B, L, H, D] tensors attention layers hold, seen as
    [B, H, L, D] through transpose(1, 2) (the kernels take the strides, no
    copy): every forward kernel gives the same bits as on contiguous
    inputs."""
    B, H, Hkv, L, Lq, D, nl, layer, w, dtype, scale = draw(700 + seed)
    print(f"strided seed={seed} B={B} H={H} Hkv={Hkv} L={L} Lq={Lq} D={D} nl={nl} "
          f"layer={layer} w={w} {dtype}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=600 + seed, scale=scale, Lq=Lq)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    qs, ks, vs = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (qd, kd, vd))
    assert torch.equal(qs, qd)
    if H > 1 and Lq > 1:
        assert qs.stride(2) > qs.stride(1)  # heads inside a row
    lay = ElasticLayout(make_pattern(L, w, layer, nl, H), DEV)
    sc = scaling_for(D)
    runs = [lambda a, b, c: elastic_attention_fwd(a, b, c, lay, sc, kernel="tile"),
            lambda a, b, c: elastic_attention_fwd(a, b, c, lay, sc, kernel="tile",
                                                  query_block=64, key_block=32),
            lambda a, b, c: elastic_attention_rows(a, b, c, lay.pattern, sc)]
    if w <= 64:
        runs.append(lambda a, b, c: elastic_attention_band(a, b, c, lay.pattern, sc))
    for run in runs:
        o1, l1 = run(qd, kd, vd)
        o2, l2 = run(qs, ks, vs)
        assert torch.equal(o1, o2) and torch.equal(l1, l2)


@pytest.mark.parametrize("seed", range(16))
def test_random_operator_explicit_indices(seed):
    """The reference operator (ElasticSparseAttentionFunction, :241-339) on
    random explicit index lists (duplicates, entries below 0 and past kv_len,
    rows with no valid entry, q_len below kv_len) at random shapes, dtypes
    and head dims: forward and gradients against autograd through the
    oracle, out-of-range entries reading a zero K / V row as the Triton
    gather mask makes them (:131-133)."""
    from elastic_sparse_attention import ElasticSparseAttentionFunction
    r = random.Random(3000 + seed)
    H = r.choice([1, 2, 4, 6])
    Hkv = r.choice([d for d in range(1, H + 1) if H % d == 0])
    L = r.randint(8, 700)
    Lq = L if r.random() < 0.5 else r.randint(1, L)
    w = r.choice([1, 5, 16, 33, 64, 90])
    D = r.choice([32, 64, 96, 128])
    dtype = r.choice([torch.float32, torch.bfloat16, torch.float16])
    B = r.choice([1, 2])
    print(f"operator seed={seed} B={B} H={H} Hkv={Hkv} L={L} Lq={Lq} w={w} D={D} {dtype}",
          flush=True)
    g = torch.Generator().manual_seed(seed)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=900 + seed, Lq=Lq)
    idx = torch.randint(-3, L + 3, (H, Lq, w), generator=g)
    if w > 1:
        idx[:, :, 1] = idx[:, :, 0]  # duplicates
    msk = (torch.rand(H, Lq, w, generator=g) > 0.25).long()
    msk[:, Lq // 2] = 0  # a row with no valid entry
    oor = (idx < 0) | (idx >= L)
    z = torch.zeros(B, Hkv, 1, D, dtype=dtype)
    k2, v2 = torch.cat([k, z], dim=2), torch.cat([v, z], dim=2)
    idx2 = torch.where(oor, torch.full_like(idx, L), idx)
    sc = D ** -0.5
    gout = torch.randn(B, H, Lq, D, generator=torch.Generator().manual_seed(7 + seed))
    qf, kf, vf = (t.detach().float().clone().requires_grad_() for t in (q, k2, v2))
    ro, _ = forward_fp32(qf, kf, vf, idx2, msk, sc, H // Hkv, chunk_rows=512)
    (ro * gout).sum().backward()
    rq, rk, rv = qf.grad, kf.grad[:, :, :L], vf.grad[:, :, :L]
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    o = ElasticSparseAttentionFunction.apply(qd, kd, vd, idx.to(DEV), msk.to(DEV), sc, H // Hkv)
    o.backward(gout.to(dtype).to(DEV))
    tol = TOL[dtype][0] if dtype != torch.float32 else 1e-4
    assert (o.detach().float().cpu() - ro.detach()).abs().max().item() <= tol
    # errors relative to each gradient's largest entry, or to 1% of dV's
    # where that is smaller: with one valid key per row (w = 1) p = 1, so
    # dS = p (dP - delta) and with it dQ and dK are exactly 0, and what the
    # kernel returns is the rounding of dP - delta
    floor = 1e-2 * rv.abs().max().item()
    e = [(x.float().cpu() - y).abs().max().item() / max(y.abs().max().item(), floor, 1e-30)
         for x, y in zip((qd.grad, kd.grad, vd.grad), (rq, rk, rv))]
    assert max(e) <= (2e-2 if dtype != torch.float32 else 1e-4), e


@pytest.mark.parametrize("seed", range(12))
def test_random_band_late_refill_order(seed):
    """The band forward's other refill order (V requested after PV), which
    the host picks where the entry spacing at the last row, (q_len a + w (1 -
    a)) / w query rows, is 1000 or more: drawn here with short attention
    lengths at the last layers, against the oracle."""
    r = random.Random(7000 + seed)
    H = r.choice([1, 2, 3, 5])
    Hkv = r.choice([d for d in range(1, H + 1) if H % d == 0])
    w = r.choice([2, 3, 4, 6, 8])
    nl = r.choice([2, 4, 8])
    layer = nl - 1 if r.random() < 0.7 else nl - 2
    a = layer / max(nl - 1, 1)
    need = int((1000 * w - w * (1 - a)) / max(a, 1e-9)) + 1 if a > 0 else None
    if need is None:
        layer, a = nl - 1, 1.0
        need = 1000 * w + 1
    L = need + r.randint(0, 2500)
    D = r.choice([64, 128])
    dtype = r.choice([torch.bfloat16, torch.float16])
    B = r.choice([1, 2])
    spacing = (torch.tensor(L, dtype=torch.float32) * torch.tensor(a, dtype=torch.float32)
               + torch.tensor(w * (1 - a), dtype=torch.float32)) / w
    assert spacing.item() >= 1000.0
    print(f"seed={seed} B={B} H={H} Hkv={Hkv} L={L} D={D} nl={nl} layer={layer} w={w} {dtype} "
          f"spacing={spacing.item():.1f}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=200 + seed, scale=D ** -0.25)
    idx, msk = elastic_indices(L, layer, nl, H, w)
    pi, pm = prepared_rows(idx, msk, L, L, L)
    sc = scaling_for(D)
    ro, rl = forward_fp32(q, k, v, pi, pm, sc, H // Hkv)
    tol, ltol = TOL[dtype]
    o, lse = elastic_attention_band(q.to(DEV), k.to(DEV), v.to(DEV),
                                    make_pattern(L, w, layer, nl, H), sc)
    check(o, lse, ro, rl, tol, ltol, "band, V after PV")
