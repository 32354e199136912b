"""HIP layout builders against the oracle (GPU): bit-exact.

esa_build_indices <- _create_elastic_sparse_indices (elastic_sparse_attention.py:470-535)
esa_build_layout  <- the block layout derived from it (oracle.block_layout)
"""
import hashlib

import pytest
import torch

from esa_oracle import block_layout, elastic_indices
from elastic_sparse_attention import ElasticLayout, build_indices, make_pattern

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().numpy().astype("<i8").tobytes()).hexdigest()


@pytest.mark.parametrize("L,H,w,nl", [(1024, 4, 64, 8), (2048, 8, 48, 8), (2048, 6, 100, 6),
                                      (300, 1, 16, 4), (200, 3, 8, 1), (333, 5, 33, 11)])
def test_indices_bit_exact_all_layers(L, H, w, nl):
    for layer in range(nl):
        print(f"indices L={L} H={H} w={w} nl={nl} layer={layer}", flush=True)
        ref_i, ref_m = elastic_indices(L, layer, nl, H, w)
        gi, gm = build_indices(make_pattern(L, w, layer, nl, H), DEV, torch.int64)
        assert torch.equal(gi.cpu(), ref_i)
        assert torch.equal(gm.cpu(), ref_m)
        gi32, gm32 = build_indices(make_pattern(L, w, layer, nl, H), DEV, torch.int32)
        assert torch.equal(gi32.cpu().long(), ref_i)
        assert torch.equal(gm32.cpu().long(), ref_m)


def test_indices_row_window():
    L, H, w = 1000, 4, 64
    ref_i, ref_m = elastic_indices(L, 5, 8, H, w)
    gi, gm = build_indices(make_pattern(L, w, 5, 8, H), DEV, torch.int64, row0=123, nrows=456)
    assert torch.equal(gi.cpu(), ref_i[:, 123:579])
    assert torch.equal(gm.cpu(), ref_m[:, 123:579])


def test_indices_match_golden_hashes(golden):
    """Every case the reference produced, including L = 32768 and 131072."""
    for c in golden["cases"]:
        print(f"golden L={c['seq_len']} H={c['heads']} layer={c['layer_idx']}", flush=True)
        p = make_pattern(c["seq_len"], c["w"], c["layer_idx"], c["layers"], c["heads"])
        gi, gm = build_indices(p, DEV, torch.int64)
        assert sha(gi.cpu()) == c["indices_sha256"], c
        assert sha(gm.cpu()) == c["mask_sha256"], c
        del gi, gm


@pytest.mark.parametrize("L,H,w,nl,layers", [(1024, 4, 64, 8, range(8)), (1000, 3, 48, 6, range(6)),
                                             (8192, 32, 64, 8, [0, 4, 7]),
                                             (4096, 16, 64, 8, [0, 4, 7])])
def test_block_layout_bit_exact(L, H, w, nl, layers):
    for layer in layers:
        print(f"layout L={L} H={H} layer={layer}", flush=True)
        idx, msk = elastic_indices(L, layer, nl, H, w)
        rp, ci = block_layout(idx, msk, 128, 128)
        lay = ElasticLayout(make_pattern(L, w, layer, nl, H), DEV)
        assert torch.equal(lay.row_ptr.cpu(), rp)
        assert torch.equal(lay.col_idx[:lay.num_tiles].cpu(), ci)


def test_block_layout_other_tiles():
    L, H, w = 1000, 3, 48
    idx, msk = elastic_indices(L, 4, 6, H, w)
    for bm, bn in [(64, 64), (128, 32), (256, 128)]:
        rp, ci = block_layout(idx, msk, bm, bn)
        lay = ElasticLayout(make_pattern(L, w, 4, 6, H, bm, bn), DEV)
        assert torch.equal(lay.row_ptr.cpu(), rp)
        assert torch.equal(lay.col_idx[:lay.num_tiles].cpu(), ci)


@pytest.mark.parametrize("L,H,layer,n", [(32768, 32, 0, 16352), (32768, 32, 4, 563523),
                                         (32768, 32, 7, 633512)])
def test_headline_layout_full_size(L, H, layer, n):
    print(f"headline layout layer={layer}", flush=True)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    rp, ci = block_layout(idx, msk, 128, 128)
    assert int(rp[-1]) == n
    lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
    assert torch.equal(lay.row_ptr.cpu(), rp)
    assert torch.equal(lay.col_idx[:lay.num_tiles].cpu(), ci)


def test_long_context_layout_full_size():
    L, H = 131072, 8
    for layer in (0, 4, 7):
        print(f"long layout layer={layer}", flush=True)
        idx, msk = elastic_indices(L, layer, 8, H, 64)
        rp, ci = block_layout(idx, msk, 128, 128)
        lay = ElasticLayout(make_pattern(L, 64, layer, 8, H), DEV)
        assert torch.equal(lay.row_ptr.cpu(), rp)
        assert torch.equal(lay.col_idx[:lay.num_tiles].cpu(), ci)
        del idx, msk


@pytest.mark.parametrize("L,H,w,nl,layer", [(700, 4, 64, 8, 0), (700, 4, 64, 8, 4),
                                            (513, 3, 33, 6, 5), (300, 1, 16, 4, 3)])
def test_module_index_buffers_and_dense_mask(L, H, w, nl, layer):
    """The reference's module surface (:454-468, :470-572): the index buffers
    are non-persistent buffers built by the HIP builders on the module's
    device, follow module.to(), and match the oracle bit for bit; the dense
    mask of implementation="dense" matches the oracle's
    _create_full_sparse_mask restatement."""
    from elastic_sparse_attention import ElasticSparseAttention
    from esa_oracle import dense_mask
    print(f"module buffers L={L} H={H} w={w} nl={nl} layer={layer}", flush=True)
    ref_i, ref_m = elastic_indices(L, layer, nl, H, w)
    m = ElasticSparseAttention(layer, nl, H, 64, w, L).to(DEV)
    assert m.state_dict() == {}
    gi, gm = m.sparse_attention_indices, m.sparse_causal_mask
    assert gi.device == DEV and gi.dtype == torch.int64 and gm.dtype == torch.int64
    assert torch.equal(gi.cpu(), ref_i) and torch.equal(gm.cpu(), ref_m)
    assert m.full_attention_mask is None
    m.to("cpu")  # built buffers follow the module
    assert m.sparse_attention_indices.device.type == "cpu"
    assert torch.equal(m.sparse_attention_indices, ref_i)
    ci, cm = m._create_elastic_sparse_indices(L - 7, torch.device("cpu"))
    assert torch.equal(ci, ref_i[:, :L - 7]) and torch.equal(cm, ref_m[:, :L - 7])
    pi, pm = m._get_prepared_indices_and_mask(L // 2)
    assert torch.equal(pi, ref_i[:, :L // 2]) and torch.equal(pm, ref_m[:, :L // 2])

    d = ElasticSparseAttention(layer, nl, H, 64, w, L, implementation="dense").to(DEV)
    assert d.sparse_attention_indices is None and d.sparse_causal_mask is None
    full = d.full_attention_mask
    assert full.shape == (1, H, L, L) and full.dtype == torch.bool and full.device == DEV
    assert torch.equal(full[0].cpu(), dense_mask(ref_i, ref_m))
    # a padded row stride: the bytes between rows are left alone
    pat = make_pattern(L, w, layer, nl, H)
    import ctypes
    from esa_native import check, load
    buf = torch.full((H, 40, L + 9), 7, dtype=torch.uint8, device=DEV)
    check(load().esa_build_dense_mask(ctypes.byref(pat), 100, 40, L,
                                      ctypes.c_void_p(buf.data_ptr()), buf.stride(0),
                                      buf.stride(1), None), "esa_build_dense_mask")
    torch.cuda.synchronize()
    b = buf.cpu()
    assert torch.equal(b[..., :L].bool(), dense_mask(ref_i, ref_m)[:, 100:140])
    assert bool((b[..., :L] <= 1).all()) and bool((b[..., L:] == 7).all())
