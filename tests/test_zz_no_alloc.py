"""esa_elastic_bwd_noalloc (the backward with the library's per-device
workspace array instead of a caller buffer) against esa_elastic_bwd (GPU).

Both run the same kernels in the same order, so the gradients must agree
bit for bit.  Two calls in a row, the second with a smaller input, so a
second call sees the array as the first left it (split partial sums and
arrival counters included: the first case splits key block 0 of the last
layer, which the kernels clear and refill on every call).
"""
import pytest
import torch

from esa_oracle import seeded_inputs
from elastic_sparse_attention import (ElasticLayout, elastic_attention_bwd, elastic_attention_fwd,
                                      make_pattern)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def grads(B, H, Hkv, L, D, layer, kernels, seed):
    q, k, v = seeded_inputs(B, H, Hkv, L, D, torch.bfloat16, seed=seed, scale=1.0)
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = elastic_attention_fwd(qd, kd, vd, lay, D ** -0.5, kernel=kernels[0])
    g = torch.Generator(device=DEV).manual_seed(seed)
    do = torch.randn(B, L, H, D, generator=g, device=DEV).to(torch.bfloat16)
    ref = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, D ** -0.5, dq_kernel=kernels[0],
                                dkdv_kernel=kernels[1])
    got = elastic_attention_bwd(qd, kd, vd, o, lse, do, lay, D ** -0.5, dq_kernel=kernels[0],
                                dkdv_kernel=kernels[1], noalloc=True)
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("kernels", [("band", "band"), ("tile", "tile")])
def test_noalloc_matches_allocating_backward(kernels):
    cases = [(1, 8, 2, 2048, 128, 7, 31),   # last layer, GQA: key block 0 split in 2 parts
             (1, 4, 4, 640, 64, 3, 32)]     # then a smaller call
    for B, H, Hkv, L, D, layer, seed in cases:
        print(f"noalloc {kernels} B={B} H={H} Hkv={Hkv} L={L} D={D} layer={layer}", flush=True)
        ref, got = grads(B, H, Hkv, L, D, layer, kernels, seed)
        for r, x in zip(ref, got):
            assert torch.equal(r, x)
            assert bool(torch.isfinite(x.float()).all())


def test_noalloc_random_sequence_of_calls():
    """A run of noalloc backward calls at seeded random shapes (every kernel
    pair, GQA, ragged lengths, decreasing and increasing sizes), each against
    the allocating entry point bit for bit: whatever one call leaves in the
    library's array, the next call's results do not depend on it."""
    import random
    r = random.Random(77)
    for step in range(12):
        H = r.choice([2, 4, 8])
        Hkv = r.choice([d for d in range(1, H + 1) if H % d == 0])
        L = r.randint(100, 2500)
        D = r.choice([64, 128])
        layer = r.randrange(8)
        kernels = r.choice([("band", "band"), ("tile", "tile"), ("band", "tile"),
                            ("tile", "band")])
        B = r.choice([1, 2])
        print(f"noalloc step {step} {kernels} B={B} H={H} Hkv={Hkv} L={L} D={D} layer={layer}",
              flush=True)
        ref, got = grads(B, H, Hkv, L, D, layer, kernels, 100 + step)
        for a, b in zip(ref, got):
            assert torch.equal(a, b)
