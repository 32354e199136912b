"""The band forward at cache_position rows (GPU): chunked prefill through the
MFMA kernel (elastic_sparse_attention.py:602-619 takes any row selection
through the same kernel).

A 16-row group whose positions are consecutive and in range runs as a
prefill group from its first position (which need not be a multiple of 16);
any other group computes its rows with the per-row gather.  Both are checked
against the float32 oracle on the rows the reference's prepared indices
select (prepared_rows, :574-615), and against the per-row gather path.
"""
import pytest
import torch

from esa_oracle import elastic_indices, forward_fp32, prepared_rows, scaling_for, seeded_inputs
from elastic_sparse_attention import (BAND_POSITION_MIN_ROWS, BAND_POSITION_MIN_UNITS,
                                      ElasticSparseAttention,
                                      elastic_attention_band, elastic_attention_rows,
                                      make_pattern)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
BF16_TOL = 2e-2
BF16_LSE_TOL = 2e-3


def check_rows(B, H, Hkv, L, D, layer, pos, dtype=torch.bfloat16, w=64, seed=5):
    """The band forward at positions pos (a host int64 tensor of in-range
    positions) against the oracle and the gather path."""
    Lq = pos.numel()
    _, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=seed, scale=1.0)
    q = seeded_inputs(B, H, Hkv, L, D, dtype, seed=seed + 1, scale=1.0, Lq=Lq)[0]
    sc = scaling_for(D)
    pat = make_pattern(L, w, layer, 8, H)
    qd, kd, vd, pd = q.to(DEV), k.to(DEV), v.to(DEV), pos.to(DEV)
    o, lse = elastic_attention_band(qd, kd, vd, pat, sc, positions=pd)
    go, glse = elastic_attention_rows(qd, kd, vd, pat, sc, pd)
    idx, msk = elastic_indices(L, layer, 8, H, w)
    pi, pm = prepared_rows(idx, msk, Lq, L, L, pos % L)
    ro, rl = forward_fp32(q, k, v, pi, pm, sc, H // Hkv)
    got = o.float().permute(0, 2, 1, 3).cpu()
    assert (got - ro).abs().max().item() <= BF16_TOL
    assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL
    assert (o.float() - go.float()).abs().max().item() <= BF16_TOL
    return o, lse


@pytest.mark.parametrize("layer,p0,Lq,D", [(4, 1000, 500, 128), (7, 37, 300, 64),
                                           (0, 1500, 548, 128), (2, 0, 256, 128),
                                           (5, 2031, 17, 64)])
def test_chunk_at_offset(layer, p0, Lq, D):
    """A chunked prefill: rows p0 .. p0 + Lq - 1 (p0 not a multiple of 16,
    ragged last group) run as band prefill groups."""
    print(f"positions chunk layer={layer} p0={p0} Lq={Lq} D={D}", flush=True)
    pos = torch.arange(p0, p0 + Lq, dtype=torch.int64)
    check_rows(1, 4, 2, 2048, D, layer, pos)


def test_chunk_matches_prefill_rows():
    """The chunk's rows agree with the same rows of a full prefill to two
    bf16 units at the outputs' magnitude: the groups cut the rows
    differently and the entry rotation follows each group's dispatch slot,
    so the bands are accumulated in another order (the running max, and with
    it P's rounding, moves at other bands)."""
    B, H, L, D, layer, p0, Lq = 1, 4, 2048, 128, 6, 777, 700
    q, k, v = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=9, scale=1.0)
    pat = make_pattern(L, 64, layer, 8, H)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    full, flse = elastic_attention_band(qd, kd, vd, pat, scaling_for(D))
    pos = torch.arange(p0, p0 + Lq, dtype=torch.int64, device=DEV)
    part, plse = elastic_attention_band(qd[:, :, p0:p0 + Lq].contiguous(), kd, vd, pat,
                                        scaling_for(D), positions=pos)
    assert (part.float() - full.float()[:, p0:p0 + Lq]).abs().max().item() <= 1e-2
    assert (plse - flse[:, :, p0:p0 + Lq]).abs().max().item() <= 1e-3


def test_mixed_and_negative_positions():
    """Groups that are not consecutive (a jump inside a group, shuffled rows,
    repeated positions) take the per-row gather; negative positions count
    from kv_len, as torch indexing does."""
    L = 1500
    g = torch.Generator().manual_seed(3)
    runs = [torch.arange(100, 140), torch.arange(700, 709), torch.tensor([5, 5, 5]),
            torch.randperm(L, generator=g)[:50], torch.arange(1480, 1500) - L]
    pos = torch.cat(runs).to(torch.int64)
    check_rows(2, 8, 2, L, 128, 5, pos)


@pytest.mark.parametrize("D", [96, 80, 40, 200])
def test_mixed_positions_padded_head_dims(D):
    """Head dims padded up to the kernel's (96 and 80 run the D = 128
    kernel, 40 the 64 one, 200 the 256 one) with groups that are not
    consecutive: those groups' rows go to the per-row gather, which must use
    the inputs' own head dim.  O is written into the front of a larger
    buffer; the elements after it must keep their sentinel (no row is
    written past its D elements)."""
    B, H, Hkv, L, layer = 2, 4, 2, 900, 5
    g = torch.Generator().manual_seed(7)
    pos = torch.cat([torch.arange(200, 248), torch.randperm(L, generator=g)[:40],
                     torch.arange(860, 900) - L]).to(torch.int64)
    Lq = pos.numel()
    _, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=9, scale=1.0)
    q = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=10, scale=1.0, Lq=Lq)[0]
    sc = scaling_for(D)
    pat = make_pattern(L, 64, layer, 8, H)
    n = B * Lq * H * D
    buf = torch.full((n + 512,), 7.0, dtype=torch.bfloat16, device=DEV)
    o = buf[:n].view(B, Lq, H, D)
    o, lse = elastic_attention_band(q.to(DEV), k.to(DEV), v.to(DEV), pat, sc, out=o,
                                    positions=pos.to(DEV))
    torch.cuda.synchronize()
    assert bool((buf[n:] == 7.0).all())
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    pi, pm = prepared_rows(idx, msk, Lq, L, L, pos % L)
    ro, rl = forward_fp32(q, k, v, pi, pm, sc, H // Hkv)
    assert (o.float().permute(0, 2, 1, 3).cpu() - ro).abs().max().item() <= BF16_TOL
    assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


def test_out_of_range_positions_give_nan_rows():
    B, H, L, D = 1, 4, 600, 64
    _, k, v = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=2, scale=1.0)
    q = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=3, scale=1.0, Lq=32)[0]
    pos = torch.arange(100, 132, dtype=torch.int64)
    pos[20] = L          # past kv_len
    pos[21] = -L - 1     # before -kv_len
    pat = make_pattern(L, 64, 3, 8, H)
    o, lse = elastic_attention_band(q.to(DEV), k.to(DEV), v.to(DEV), pat, scaling_for(D),
                                    positions=pos.to(DEV))
    bad = torch.zeros(32, dtype=torch.bool)
    bad[20:22] = True
    assert bool(torch.isnan(o.float()[:, bad]).all()) and bool(torch.isnan(lse[:, :, bad]).all())
    assert bool(torch.isfinite(o.float()[:, ~bad]).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_module_chunked_prefill(dtype):
    """ElasticSparseAttention.forward with a device cache_position of at least
    BAND_POSITION_MIN_ROWS rows and more than BAND_POSITION_MIN_UNITS * 128 /
    head_dim (batch, head, row) units runs the band kernel; its output and its gradients (the
    gather backward at the same positions) match the oracle and torch
    autograd through it."""
    B, H, Hkv, L, D, layer, p0, Lq = 2, 8, 2, 1024, 128, 4, 333, 300
    assert Lq >= BAND_POSITION_MIN_ROWS and B * H * Lq * D > BAND_POSITION_MIN_UNITS * 128
    m = ElasticSparseAttention(layer, 8, H, D, 64, L, num_key_value_heads=Hkv)
    _, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=11, scale=1.0)
    q = seeded_inputs(B, H, Hkv, L, D, dtype, seed=12, scale=1.0, Lq=Lq)[0]
    pos = torch.arange(p0, p0 + Lq, dtype=torch.int64)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out, _ = m(qd, kd, vd, cache_position=pos.to(DEV))
    g = torch.randn(B, Lq, H * D, generator=torch.Generator().manual_seed(1)).to(dtype)
    out.backward(g.to(DEV))
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    pi, pm = prepared_rows(idx, msk, Lq, L, L, pos)
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    ro, _ = forward_fp32(qf, kf, vf, pi, pm, m.scaling, H // Hkv)
    ro = ro.transpose(1, 2).reshape(B, Lq, H * D)
    (ro * g.float()).sum().backward()
    assert (out.detach().float().cpu() - ro.detach()).abs().max().item() <= BF16_TOL
    for got, ref in ((qd.grad, qf.grad), (kd.grad, kf.grad), (vd.grad, vf.grad)):
        err = (got.float().cpu() - ref).abs().max().item()
        assert err <= 2e-2 * ref.abs().max().item(), err


@pytest.mark.parametrize("p0,Lq,D,w", [(1500, 548, 128, 64), (37, 300, 64, 64), (0, 100, 128, 17),
                                       (2000, 48, 64, 48)])
def test_window_chunk_at_offset(p0, Lq, D, w):
    """Layer 0 (the sliding-window kernel) at cache_position rows: 32-row
    groups of consecutive positions from p0 (not a multiple of 16, ragged
    last group) run from their first position."""
    print(f"window positions p0={p0} Lq={Lq} D={D} w={w}", flush=True)
    pos = torch.arange(p0, p0 + Lq, dtype=torch.int64)
    check_rows(1, 4, 2, 2048, D, 0, pos, w=w)


def test_window_mixed_and_negative_positions():
    """Layer 0: groups that are not consecutive take the per-row gather
    (a jump inside a 32-row group, repeated and shuffled positions), and
    negative positions count from kv_len."""
    L = 1500
    g = torch.Generator().manual_seed(4)
    runs = [torch.arange(100, 150), torch.arange(700, 714), torch.tensor([5, 5, 5]),
            torch.randperm(L, generator=g)[:40], torch.arange(1470, 1500) - L]
    pos = torch.cat(runs).to(torch.int64)
    check_rows(2, 8, 2, L, 128, 0, pos)
