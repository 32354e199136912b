"""HIP graph capture of the boundary (GPU).

The module's prefill forward (band and tile kernels) and the allocation-free
backward entry point (esa_elastic_bwd_noalloc, for callers that record
graphs) are recorded in a torch.cuda.CUDAGraph after eager warm-up calls
(which build the layout, work lists, stage masks and backward plans; the
library's per-device workspace address is looked up by esa_init_device),
then replayed.  Each replay runs on
new input contents written into the recorded (static) tensors, with eager
work and synchronisations between replays, and must give the same bits as an
eager call on the same inputs: every kernel on these paths is deterministic,
and none is preceded by a memset (the counters the backward uses are cleared
by its first kernel).
"""
import pytest
import torch

from esa_oracle import scaling_for, seeded_inputs
from elastic_sparse_attention import (ElasticLayout, ElasticSparseAttention, elastic_attention_bwd,
                                      elastic_attention_fwd, init_device, make_pattern)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def inputs(B, H, Hkv, L, D, seed):
    return [t.to(DEV) for t in seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=seed,
                                             scale=1.0)]


def warm_up(fn):
    """Eager calls on a side stream before capture, as torch.cuda.graph expects."""
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()


@pytest.mark.parametrize("kernel,layer,L,H,D", [("band", 4, 2048, 8, 128), ("tile", 4, 2048, 8, 128),
                                                ("tile", 0, 1024, 4, 128), ("tile", 2, 1024, 4, 64),
                                                ("band", 7, 1536, 4, 64),
                                                ("band", 0, 1024, 4, 128)])
def test_module_forward_graph_replays(kernel, layer, L, H, D):
    print(f"graph forward {kernel} layer={layer} L={L} H={H} D={D}", flush=True)
    m = ElasticSparseAttention(layer, 8, H, D, 64, L)
    m.prefill_kernel = kernel
    q, k, v = inputs(1, H, H, L, D, seed=layer)
    with torch.no_grad():
        warm_up(lambda: m(q, k, v))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out, _ = m(q, k, v)
        for rep in range(3):
            nq, nk, nv = inputs(1, H, H, L, D, seed=100 + rep)
            q.copy_(nq)
            k.copy_(nk)
            v.copy_(nv)
            g.replay()
            torch.cuda.synchronize()
            ref, _ = m(nq, nk, nv)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), rep


def test_noalloc_first_call_captured_after_init():
    """esa_init_device at set-up, then the process's first allocation-free
    backward is itself captured (no eager noalloc call before it: the
    eager warm-up below uses the allocating entry point, which builds the
    plans and masks).  Runs before every other noalloc test of the suite (the
    test files run in name order and this is the first noalloc test here), so
    the capture holds the entry point's first call on the device."""
    print("graph noalloc first call after esa_init_device", flush=True)
    B, H, Hkv, L, D, layer = 1, 4, 4, 1024, 128, 5
    sc = scaling_for(D)
    init_device(DEV)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    q, k, v = inputs(B, H, Hkv, L, D, seed=41)
    gen = torch.Generator(device="cpu").manual_seed(41)
    do = torch.randn(B, L, H, D, generator=gen).to(torch.bfloat16).to(DEV)
    o, lse = elastic_attention_fwd(q, k, v, lay, sc, kernel="tile")

    def bwd(noalloc):
        return elastic_attention_bwd(q, k, v, o, lse, do, lay, sc, dq_kernel="tile",
                                     dkdv_kernel="tile", noalloc=noalloc)

    warm_up(lambda: bwd(False))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dq, dk, dv = bwd(True)
    for rep in range(2):
        g.replay()
        torch.cuda.synchronize()
        rq, rk, rv = bwd(False)
        torch.cuda.synchronize()
        assert torch.equal(dq, rq) and torch.equal(dk, rk) and torch.equal(dv, rv), rep


@pytest.mark.parametrize("kernel,layer,L,H,Hkv,D", [("band", 4, 2048, 8, 8, 128),
                                                    ("tile", 3, 1024, 4, 2, 64),
                                                    ("band", 7, 2048, 4, 4, 128),
                                                    ("tile", 7, 1024, 4, 4, 128),
                                                    ("band", 0, 1024, 4, 2, 128)])
def test_noalloc_backward_graph_replays(kernel, layer, L, H, Hkv, D):
    print(f"graph noalloc backward {kernel} layer={layer} L={L} H={H} Hkv={Hkv} D={D}", flush=True)
    B = 1
    sc = scaling_for(D)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    q, k, v = inputs(B, H, Hkv, L, D, seed=layer + 1)
    g0 = torch.Generator(device="cpu").manual_seed(layer)
    do = torch.randn(B, L, H, D, generator=g0).to(torch.bfloat16).to(DEV)
    o, lse = elastic_attention_fwd(q, k, v, lay, sc, kernel=kernel)

    def bwd(noalloc):
        return elastic_attention_bwd(q, k, v, o, lse, do, lay, sc, dq_kernel=kernel,
                                     dkdv_kernel=kernel, noalloc=noalloc)

    warm_up(lambda: bwd(True))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dq, dk, dv = bwd(True)
    for rep in range(3):
        nq, nk, nv = inputs(B, H, Hkv, L, D, seed=200 + rep)
        gen = torch.Generator(device="cpu").manual_seed(300 + rep)
        ndo = torch.randn(B, L, H, D, generator=gen).to(torch.bfloat16).to(DEV)
        no, nlse = elastic_attention_fwd(nq, nk, nv, lay, sc, kernel=kernel)
        for dst, src in ((q, nq), (k, nk), (v, nv), (do, ndo), (o, no), (lse, nlse)):
            dst.copy_(src)
        g.replay()
        torch.cuda.synchronize()
        rq, rk, rv = elastic_attention_bwd(nq, nk, nv, no, nlse, ndo, lay, sc, dq_kernel=kernel,
                                           dkdv_kernel=kernel)
        torch.cuda.synchronize()
        assert torch.equal(dq, rq) and torch.equal(dk, rk) and torch.equal(dv, rv), rep
