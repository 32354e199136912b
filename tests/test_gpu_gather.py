"""Gather paths on the GPU: the reference operator's backward over explicit
index lists, the module's float32 / float16 / other-head_dim / decode paths
with their backward, the naive path's attention weights and dropout.

References: torch autograd through the float32 oracle forward
(oracle/esa_oracle.py forward_fp32, pinned against dense brute force and
SDPA) for gradients; the oracle forward for outputs and weights.  Bars:
float32 1e-4 (outputs) and 1e-4 x max |reference| (gradients); bfloat16 and
float16 2e-2 (outputs) and 2e-2 x max |reference| (gradients).  The gather
backward sums every gradient element in one wave in a fixed order, so two
runs agree bit for bit.
"""
import pytest
import torch

from esa_oracle import elastic_indices, forward_fp32, prepared_rows, scaling_for, seeded_inputs
from elastic_sparse_attention import (ElasticSparseAttention, ElasticSparseAttentionFunction,
                                      elastic_attention_bwd_rows, elastic_attention_rows,
                                      make_pattern, sparse_attention_bwd, sparse_attention_fwd)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def rel_err(got, ref):
    return ((got.float().cpu() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def oracle_grads(q, k, v, idx, msk, sc, groups, g):
    # (a copy: .float() of a float32 tensor is the tensor itself)
    qf, kf, vf = (t.detach().float().clone().requires_grad_() for t in (q, k, v))
    o, _ = forward_fp32(qf, kf, vf, idx, msk, sc, groups, chunk_rows=512)
    (o * g).sum().backward()
    return o.detach(), qf.grad, kf.grad, vf.grad


def explicit_case(B, H, Hkv, L, D, w, dtype, seed):
    """Random index lists with duplicates, out-of-range entries, empty rows,
    and the oracle's view of them (out-of-range entries read a zero row
    appended to K and V, as the Triton gather mask makes them, :131-133)."""
    g = torch.Generator().manual_seed(seed)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=seed)
    idx = torch.randint(-3, L + 3, (H, L, w), generator=g)
    idx[:, :, 1] = idx[:, :, 0]          # duplicates
    msk = (torch.rand(H, L, w, generator=g) > 0.25).long()
    msk[:, 5] = 0                        # empty rows
    oor = (idx < 0) | (idx >= L)
    z = torch.zeros(B, Hkv, 1, D, dtype=dtype)
    k2, v2 = torch.cat([k, z], dim=2), torch.cat([v, z], dim=2)
    idx2 = torch.where(oor, torch.full_like(idx, L), idx)
    return q, k, v, idx, msk, k2, v2, idx2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,Hkv,L,D,w", [(2, 4, 2, 300, 64, 24), (1, 3, 1, 130, 128, 70),
                                           (1, 2, 2, 64, 96, 8)])
def test_operator_backward_matches_autograd(dtype, B, H, Hkv, L, D, w):
    """ElasticSparseAttentionFunction.backward (:299-339) on arbitrary index
    lists: dq, dk, dv against autograd through the oracle."""
    print(f"operator bwd {dtype} B={B} H={H} Hkv={Hkv} L={L} D={D} w={w}", flush=True)
    q, k, v, idx, msk, k2, v2, idx2 = explicit_case(B, H, Hkv, L, D, w, dtype, seed=D + w)
    sc = 0.3
    gout = torch.randn(B, H, L, D, generator=torch.Generator().manual_seed(9))
    ro, rq, rk2, rv2 = oracle_grads(q, k2, v2, idx2, msk, sc, H // Hkv, gout)
    rk, rv = rk2[:, :, :L], rv2[:, :, :L]
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    o = ElasticSparseAttentionFunction.apply(qd, kd, vd, idx.to(DEV), msk.to(DEV), sc, H // Hkv)
    o.backward(gout.to(dtype).to(DEV))
    tol = TOL[dtype]
    assert (o.detach().float().cpu() - ro).abs().max().item() <= tol
    e = (rel_err(qd.grad, rq), rel_err(kd.grad, rk), rel_err(vd.grad, rv))
    print(f"  rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert max(e) <= tol
    assert qd.grad.dtype == dtype and kd.grad.shape == k.shape
    # rows with no valid entry get no gradient; deterministic reruns
    assert torch.equal(qd.grad[:, :, 5].float().cpu(), torch.zeros(B, H, D))
    o2, lse2 = sparse_attention_fwd(qd.detach(), kd.detach(), vd.detach(), idx.to(DEV),
                                    msk.to(DEV), sc, H // Hkv)
    g1 = sparse_attention_bwd(qd.detach(), kd.detach(), vd.detach(), o2, lse2,
                              gout.to(dtype).to(DEV), idx.to(DEV), msk.to(DEV), sc)
    g2 = sparse_attention_bwd(qd.detach(), kd.detach(), vd.detach(), o2, lse2,
                              gout.to(dtype).to(DEV), idx.to(DEV), msk.to(DEV), sc)
    assert all(torch.equal(a, b) for a, b in zip(g1, g2))


def test_operator_backward_reference_indices_full_layer():
    """The operator on the module's own index buffers (prepared as
    _triton_forward prepares them, :600-615) at L = 2048, last layer, GQA,
    bf16: the path a caller of the reference's Function takes."""
    B, H, Hkv, L, D, layer = 1, 8, 2, 2048, 128, 7
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=3, scale=1.0)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    pi, pm = prepared_rows(idx, msk, L, L, L)
    gout = torch.randn(B, H, L, D, generator=torch.Generator().manual_seed(1))
    _, rq, rk, rv = oracle_grads(q, k, v, pi, pm, D ** -0.5, H // Hkv, gout)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    o = ElasticSparseAttentionFunction.apply(qd, kd, vd, pi.to(DEV), pm.to(DEV), D ** -0.5,
                                             H // Hkv)
    o.backward(gout.to(torch.bfloat16).to(DEV))
    e = (rel_err(qd.grad, rq), rel_err(kd.grad, rk), rel_err(vd.grad, rv))
    print(f"  operator full layer rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert max(e) <= 2e-2


@pytest.mark.parametrize("dtype,D", [(torch.float32, 64), (torch.float16, 128),
                                     (torch.bfloat16, 96), (torch.float32, 36)])
def test_module_rows_backward(dtype, D):
    """The module's gather path (float32, float16, head dims the MFMA kernels
    do not take) forward and backward against the oracle."""
    B, H, Hkv, L, layer = 2, 4, 2, 700, 5
    print(f"module rows {dtype} D={D}", flush=True)
    m = ElasticSparseAttention(layer, 8, H, D, 64, 1024, num_key_value_heads=Hkv)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, dtype, seed=D, scale=1.0)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    gout = torch.randn(B, L, H * D, generator=torch.Generator().manual_seed(4))
    gref = gout.view(B, L, H, D).permute(0, 2, 1, 3)
    ro, rq, rk, rv = oracle_grads(q, k, v, idx, msk, m.scaling, H // Hkv, gref)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out, wts = m(qd, kd, vd)
    assert wts is None and out.dtype == dtype
    out.backward(gout.to(dtype).to(DEV))
    tol = TOL[dtype]
    ref = ro.permute(0, 2, 1, 3).reshape(B, L, H * D)
    assert (out.detach().float().cpu() - ref).abs().max().item() <= tol
    e = (rel_err(qd.grad, rq), rel_err(kd.grad, rk), rel_err(vd.grad, rv))
    print(f"  rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert max(e) <= tol


def test_module_decode_backward():
    """Decode rows (cache_position) backpropagate into the cache: gradients
    against autograd through the oracle on the selected rows."""
    B, H, Hkv, L, D, layer = 1, 4, 4, 500, 128, 6
    m = ElasticSparseAttention(layer, 8, H, D, 64, 512)
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.float32, seed=8, scale=1.0)
    pos = torch.tensor([499, 17, 250, 63])
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    pi, pm = prepared_rows(idx, msk, len(pos), L, L, cache_position=pos)
    qs = q[:, :, pos]
    gout = torch.randn(B, len(pos), H * D, generator=torch.Generator().manual_seed(2))
    gref = gout.view(B, len(pos), H, D).permute(0, 2, 1, 3)
    ro, rq, rk, rv = oracle_grads(qs, k, v, pi, pm, m.scaling, 1, gref)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (qs.contiguous(), k, v))
    out, _ = m(qd, kd, vd, cache_position=pos.to(DEV))
    out.backward(gout.to(DEV))
    e = (rel_err(qd.grad, rq), rel_err(kd.grad, rk), rel_err(vd.grad, rv))
    print(f"  decode rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert max(e) <= 1e-4


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_naive_path_returns_weights(dtype):
    """implementation="naive" returns the attention weights [B, H, Lq, w]
    (:673-680): softmax over each row's valid entries, 0 at masked entries,
    and the output is the weighted sum of the gathered values."""
    B, H, L, D, layer, w = 1, 4, 300, 64, 3, 64
    m = ElasticSparseAttention(layer, 8, H, D, w, 512, implementation="naive")
    q, k, v = seeded_inputs(B, H, H, L, D, dtype, seed=5, scale=1.0)
    idx, msk = elastic_indices(L, layer, 8, H, w)
    with torch.no_grad():
        out, wts = m(q.to(DEV), k.to(DEV), v.to(DEV))
    assert wts.shape == (B, H, L, w) and wts.dtype == dtype
    qf, kf = q.float(), k.float()
    gk = torch.take_along_dim(kf.unsqueeze(2), idx.unsqueeze(0).unsqueeze(-1), dim=3)
    s = (qf.unsqueeze(3) * gk).sum(-1) * m.scaling
    s = s.masked_fill(msk.unsqueeze(0) < 1, float("-inf"))
    ref_w = torch.softmax(s, dim=-1)
    assert (wts.float().cpu() - ref_w).abs().max().item() <= TOL[dtype]
    assert bool((wts.float().cpu()[msk.unsqueeze(0).expand_as(wts) == 0] == 0).all())
    ro, _ = forward_fp32(q, k, v, idx, msk, m.scaling, 1)
    assert (out.float().cpu() - ro.permute(0, 2, 1, 3).reshape(B, L, H * D)).abs().max().item() \
        <= TOL[dtype]


def test_naive_dropout_training():
    """Training-mode dropout on the naive path (:674): weights are 0 or
    p / (1 - p_drop) per entry with about p_drop of the valid entries
    dropped, the output is the weighted sum of the gathered values under
    exactly those weights, eval mode drops nothing, and the backward equals
    autograd through that weighted sum with the kernel's keep mask fixed."""
    B, H, L, D, layer, w, p = 2, 4, 400, 64, 4, 64, 0.3
    m = ElasticSparseAttention(layer, 8, H, D, w, 512, attention_dropout=p,
                               implementation="naive")
    m.train()
    q, k, v = seeded_inputs(B, H, H, L, D, torch.float32, seed=12, scale=1.0)
    idx, msk = elastic_indices(L, layer, 8, H, w)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    torch.manual_seed(7)
    out, wts = m(qd, kd, vd)
    valid = msk.bool().unsqueeze(0).expand(B, H, L, w)
    wc = wts.detach().cpu()
    keep = (wc != 0) & valid
    frac = 1.0 - keep.sum().item() / valid.sum().item()
    assert abs(frac - p) < 0.02, frac
    # kept weights are the softmax probabilities scaled by 1 / (1 - p)
    qf, kf, vf = (t.detach().clone().requires_grad_() for t in (q, k, v))
    gk = torch.take_along_dim(kf.unsqueeze(2), idx.unsqueeze(0).unsqueeze(-1), dim=3)
    gv = torch.take_along_dim(vf.unsqueeze(2), idx.unsqueeze(0).unsqueeze(-1), dim=3)
    s = (qf.unsqueeze(3) * gk).sum(-1) * m.scaling
    s = s.masked_fill(~valid, float("-inf"))
    pw = torch.softmax(s, dim=-1) * keep.float() / (1.0 - p)
    assert (wc - pw.detach()).abs().max().item() <= 1e-4
    ref = (pw.unsqueeze(-1) * gv).sum(3)
    refo = ref.permute(0, 2, 1, 3).reshape(B, L, H * D)
    assert (out.detach().cpu() - refo.detach()).abs().max().item() <= 1e-4
    g = torch.randn(B, L, H * D, generator=torch.Generator().manual_seed(3))
    out.backward(g.to(DEV))
    (refo * g).sum().backward()
    e = (rel_err(qd.grad, qf.grad), rel_err(kd.grad, kf.grad), rel_err(vd.grad, vf.grad))
    print(f"  dropout bwd rel err dq {e[0]:.3e} dk {e[1]:.3e} dv {e[2]:.3e}", flush=True)
    assert max(e) <= 1e-4
    # the same seed gives the same mask; eval mode drops nothing
    torch.manual_seed(7)
    with torch.no_grad():
        _, wts2 = m(qd.detach(), kd.detach(), vd.detach())
    assert torch.equal(wts2, wts.detach())
    m.eval()
    with torch.no_grad():
        _, wts3 = m(qd.detach(), kd.detach(), vd.detach())
    assert bool((wts3.cpu()[valid] != 0).all())


def test_rows_backward_functional_matches_module():
    """elastic_attention_bwd_rows called directly equals the module's
    autograd result bit for bit (same kernels, fixed summation order)."""
    B, H, L, D, layer = 1, 2, 256, 128, 2
    q, k, v = seeded_inputs(B, H, H, L, D, torch.float16, seed=1, scale=1.0)
    pat = make_pattern(L, 64, layer, 8, H)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_rows(qd, kd, vd, pat, D ** -0.5)
    do = torch.randn(B, L, H, D, generator=torch.Generator().manual_seed(0)).half().to(DEV)
    a = elastic_attention_bwd_rows(qd, kd, vd, o, lse, do, pat, D ** -0.5)
    b = elastic_attention_bwd_rows(qd, kd, vd, o, lse, do, pat, D ** -0.5)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    assert all(bool(torch.isfinite(x.float()).all()) for x in a)
