"""float16 through the MFMA kernels (GPU): the band and block-sparse
forwards and their backward on v_mfma_*_f16, against the float32 oracle.

The reference loads any float type and computes in float32, storing in the
output's dtype (elastic_sparse_attention.py:114, :163).  Here the QK^T and
PV products take float16 operands (inputs as stored, P rounded to float16)
with float32 accumulation.  Bars as for bfloat16: output max-abs <= 2e-2,
lse <= 2e-3, gradients <= 2e-2 x max |reference| per tensor; float16 keeps
three more mantissa bits than bfloat16, so the measured errors are smaller.
"""
import pytest
import torch

from esa_oracle import elastic_indices, forward_fp32, prepared_rows, scaling_for, seeded_inputs
from elastic_sparse_attention import (ElasticLayout, ElasticSparseAttention, elastic_attention_bwd,
                                      elastic_attention_fwd, make_pattern)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TOL, LSE_TOL = 2e-2, 2e-3


def rel_err(got, ref):
    return ((got.float().cpu() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("kernel", ["band", "tile"])
@pytest.mark.parametrize("D", [128, 64])
def test_fp16_forward_all_layers(kernel, D):
    B, H, Hkv, L, Lq = 2, 4, 2, 1000, 931
    for layer in range(8):
        print(f"fp16 fwd {kernel} D={D} layer={layer}", flush=True)
        q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.float16, seed=layer, scale=1.0, Lq=Lq)
        idx, msk = elastic_indices(L, layer, 8, H, 64)
        pi, pm = prepared_rows(idx, msk, Lq, L, L)
        sc = scaling_for(D)
        lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
        o, lse = elastic_attention_fwd(q.to(DEV), k.to(DEV), v.to(DEV), lay, sc, kernel=kernel)
        assert o.dtype == torch.float16
        ro, rl = forward_fp32(q, k, v, pi, pm, sc, H // Hkv)
        e_o = (o.permute(0, 2, 1, 3).float().cpu() - ro).abs().max().item()
        e_l = (lse.cpu() - rl).abs().max().item()
        assert e_o <= TOL and e_l <= LSE_TOL, (e_o, e_l)


@pytest.mark.parametrize("kernels", ["band/band", "tile/tile", "band/tile", "tile/band"])
@pytest.mark.parametrize("B,H,Hkv,L,D,layer", [(1, 4, 4, 1024, 128, 4), (2, 8, 2, 640, 64, 7),
                                               (1, 4, 2, 700, 128, 0)])
def test_fp16_backward_matches_autograd(kernels, B, H, Hkv, L, D, layer):
    dq_kernel, dkdv_kernel = kernels.split("/")
    print(f"fp16 bwd {kernels} B={B} H={H} Hkv={Hkv} L={L} D={D} layer={layer}", flush=True)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.float16, seed=layer + 1, scale=1.0)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    sc = scaling_for(D)
    g = torch.randn(B, H, L, D, generator=torch.Generator().manual_seed(layer))
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    ro, _ = forward_fp32(qf, kf, vf, idx, msk, sc, H // Hkv, chunk_rows=512)
    (ro * g).sum().backward()
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, sc)
    do = g.half().to(DEV).permute(0, 2, 1, 3).contiguous()
    dq, dk, dv = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel=dq_kernel,
                                       dkdv_kernel=dkdv_kernel)
    assert dq.dtype == torch.float16
    e = (rel_err(dq, qf.grad), rel_err(dk, kf.grad), rel_err(dv, vf.grad))
    print(f"  rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert max(e) <= TOL
    dq2, dk2, dv2 = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, sc, dq_kernel=dq_kernel,
                                          dkdv_kernel=dkdv_kernel)
    assert torch.equal(dq, dq2) and torch.equal(dk, dk2) and torch.equal(dv, dv2)


def test_fp16_module_autograd():
    """The drop-in module with float16 inputs runs the MFMA kernels forward
    and backward."""
    B, H, L, D, layer = 1, 4, 768, 128, 5
    m = ElasticSparseAttention(layer, 8, H, D, 64, 1024)
    q, k, v = seeded_inputs(B, H, H, L, D, torch.float16, seed=4, scale=1.0)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    g = torch.randn(B, L, H * D, generator=torch.Generator().manual_seed(1))
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out, _ = m(qd, kd, vd)
    assert out.dtype == torch.float16
    out.backward(g.half().to(DEV))
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    ro, _ = forward_fp32(qf, kf, vf, idx, msk, m.scaling, 1)
    ref = ro.permute(0, 2, 1, 3).reshape(B, L, H * D)
    (ref * g).sum().backward()
    assert (out.detach().float().cpu() - ref.detach()).abs().max().item() <= TOL
    e = (rel_err(qd.grad, qf.grad), rel_err(kd.grad, kf.grad), rel_err(vd.grad, vf.grad))
    print(f"  fp16 module rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert max(e) <= TOL
