"""The band forward at head dims other than 64 and 128 (GPU): D = 256 on its
own kernel, and any other multiple of 8 up to 256 through the next of 64,
128, 256 with zero padding (the reference kernel takes any power-of-two
HEAD_DIM, elastic_sparse_attention.py:74, :94, :114).  Against the float32
oracle (forward_fp32, :624-680), through the module too, whose gradients at
these dims come from the gather backward."""
import pytest
import torch

from esa_oracle import elastic_indices, forward_fp32, prepared_rows, scaling_for, seeded_inputs
from elastic_sparse_attention import (ElasticSparseAttention, elastic_attention_band,
                                      make_pattern)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
BF16_TOL = 2e-2
BF16_LSE_TOL = 2e-3


@pytest.mark.parametrize("D,layer,dtype", [(256, 4, torch.bfloat16), (256, 7, torch.float16),
                                           (256, 0, torch.bfloat16), (96, 4, torch.bfloat16),
                                           (80, 6, torch.float16), (192, 2, torch.bfloat16),
                                           (32, 5, torch.bfloat16), (160, 1, torch.bfloat16),
                                           (8, 3, torch.bfloat16)])
def test_band_head_dims_against_oracle(D, layer, dtype):
    print(f"band head_dim D={D} layer={layer} {dtype}", flush=True)
    B, H, Hkv, L, w = 2, 4, 2, 777, 64
    q, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=D + layer, scale=1.0)
    sc = scaling_for(D)
    pat = make_pattern(L, w, layer, 8, H)
    o, lse = elastic_attention_band(q.to(DEV), k.to(DEV), v.to(DEV), pat, sc)
    idx, msk = elastic_indices(L, layer, 8, H, w)
    ro, rl = forward_fp32(q, k, v, idx, msk, sc, H // Hkv)
    assert (o.float().permute(0, 2, 1, 3).cpu() - ro).abs().max().item() <= BF16_TOL
    assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


def test_band_d256_positions():
    """D = 256 at cache_position rows: a chunk and a shuffled group."""
    B, H, L, D, layer = 1, 4, 1200, 256, 5
    pos = torch.cat([torch.arange(500, 580), torch.tensor([3, 900, 17, 1199])])
    _, k, v = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=8, scale=1.0)
    q = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=9, scale=1.0, Lq=pos.numel())[0]
    sc = scaling_for(D)
    o, lse = elastic_attention_band(q.to(DEV), k.to(DEV), v.to(DEV), make_pattern(L, 64, layer, 8, H),
                                    sc, positions=pos.to(DEV))
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    pi, pm = prepared_rows(idx, msk, pos.numel(), L, L, pos)
    ro, rl = forward_fp32(q, k, v, pi, pm, sc, 1)
    assert (o.float().permute(0, 2, 1, 3).cpu() - ro).abs().max().item() <= BF16_TOL
    assert (lse.cpu() - rl).abs().max().item() <= BF16_LSE_TOL


@pytest.mark.parametrize("D", [256, 96])
def test_module_head_dims_forward_and_grad(D):
    B, H, L, layer = 1, 4, 600, 3
    m = ElasticSparseAttention(layer, 8, H, D, 64, L)
    q, k, v = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=21, scale=1.0)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out, _ = m(qd, kd, vd)
    g = torch.randn(B, L, H * D, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    out.backward(g.to(DEV))
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    ro, _ = forward_fp32(qf, kf, vf, idx, msk, m.scaling, 1)
    ro = ro.transpose(1, 2).reshape(B, L, H * D)
    (ro * g.float()).sum().backward()
    assert (out.detach().float().cpu() - ro.detach()).abs().max().item() <= BF16_TOL
    for got, ref in ((qd.grad, qf.grad), (kd.grad, kf.grad), (vd.grad, vf.grad)):
        assert (got.float().cpu() - ref).abs().max().item() <= 2e-2 * ref.abs().max().item()
