"""The C ABI on the CPU: the library loads, exports every entry point
include/esa.h declares, rejects invalid arguments on the host with the
documented status codes (nothing is launched), and plans LPT work lists.
No test here calls a kernel."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

import esa_native as en
from esa_oracle import block_layout, elastic_indices

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions(name="esa.h"):
    text = open(os.path.join(ROOT, "include", name)).read()
    return re.findall(r"^(?:esa_status|const char\*|size_t)\s+(esa_\w+)\(", text, re.M)


def test_library_exports_header_symbols():
    lib = en.load()
    names = header_functions()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(en.EXPORTED)
    assert lib.esa_version().decode().startswith("esa-gfx950")
    assert lib.esa_status_string(en.ESA_ERR_ALIGN).decode() == "misaligned pointer or stride"


def test_probe_library_exports_and_rejects():
    """libesa_probe.so exports what include/esa_probe.h declares and checks
    its arguments on the host (nothing is launched)."""
    lib = en.load_probe()
    names = header_functions("esa_probe.h")
    assert set(names) == set(en.PROBE_EXPORTED)
    fake = ctypes.c_void_p(4096)
    assert lib.esa_probe_mfma_bf16(8, 16, 0x3f80, None, 2048, None) == en.ESA_ERR_NULL
    assert lib.esa_probe_mfma_bf16(0, 16, 0x3f80, fake, 2048, None) == en.ESA_ERR_SHAPE
    assert lib.esa_probe_mfma_bf16(8, 16385, 0x3f80, fake, 2048, None) == en.ESA_ERR_SHAPE
    assert lib.esa_probe_mfma_bf16(8, 16, 0x3f80, fake, 2047, None) == en.ESA_ERR_CAPACITY
    assert lib.esa_probe_l2_to_lds(fake, 16384 * 3 + 1, 8, 4, 7, fake, 2048, None) \
        == en.ESA_ERR_SHAPE
    assert lib.esa_probe_l2_to_lds(fake, 1 << 31, 8, 4, 7, fake, 2048, None) == en.ESA_ERR_SHAPE
    assert lib.esa_probe_l2_to_lds(fake, 16384, 8, 4, -1, fake, 2048, None) == en.ESA_ERR_SHAPE
    assert lib.esa_probe_l2_to_lds(ctypes.c_void_p(4100), 16384, 8, 4, 7, fake, 2048, None) \
        == en.ESA_ERR_ALIGN
    assert lib.esa_probe_l2_to_lds(fake, 16384, 8, 4, 7, fake, 100, None) == en.ESA_ERR_CAPACITY
    assert lib.esa_probe_hbm_read(fake, 100, 8, fake, 2048, None) == en.ESA_ERR_SHAPE
    assert lib.esa_probe_hbm_read(None, 128, 8, fake, 2048, None) == en.ESA_ERR_NULL
    assert lib.esa_probe_hbm_read(fake, 128, 8, fake, 2047, None) == en.ESA_ERR_CAPACITY
    assert lib.esa_probe_gather_to_lds(fake, 100, fake, 100, 8, 4, fake, 2048, None) \
        == en.ESA_ERR_SHAPE
    assert lib.esa_probe_gather_to_lds(fake, 1 << 23, fake, 128, 8, 4, fake, 2048, None) \
        == en.ESA_ERR_SHAPE
    assert lib.esa_probe_gather_to_lds(fake, 100, ctypes.c_void_p(4096 + 32), 128, 8, 4, fake,
                                       2048, None) == en.ESA_ERR_ALIGN
    assert lib.esa_probe_gather_to_lds(fake, 100, fake, 128, 8, 4, fake, 2047, None) \
        == en.ESA_ERR_CAPACITY
    assert lib.esa_probe_gather_read(fake, 0, fake, 10, 8, fake, 2048, None) == en.ESA_ERR_SHAPE
    assert lib.esa_probe_gather_read(fake, 10, None, 10, 8, fake, 2048, None) == en.ESA_ERR_NULL
    assert lib.esa_probe_gather_read(fake, 10, ctypes.c_void_p(4098), 10, 8, fake, 2048, None) \
        == en.ESA_ERR_ALIGN
    assert lib.esa_probe_gather_read(fake, 10, fake, 10, 8, fake, 2047, None) \
        == en.ESA_ERR_CAPACITY
    assert lib.esa_probe_lds_read(0, 8, 4, None, 2048, None) == en.ESA_ERR_NULL
    assert lib.esa_probe_lds_read(4, 8, 4, fake, 2048, None) == en.ESA_ERR_SHAPE
    assert lib.esa_probe_lds_read(-1, 8, 4, fake, 2048, None) == en.ESA_ERR_SHAPE
    assert lib.esa_probe_lds_read(1, 0, 4, fake, 2048, None) == en.ESA_ERR_SHAPE
    assert lib.esa_probe_lds_read(1, 8, 0, fake, 2048, None) == en.ESA_ERR_SHAPE
    assert lib.esa_probe_lds_read(2, 8, 4, fake, 2047, None) == en.ESA_ERR_CAPACITY


def pat(L=32768, w=64, layer=4, nl=8, H=32, bm=128, bn=128):
    return en.EsaPattern(L, w, layer, nl, H, bm, bn)


def test_layout_sizes():
    lib = en.load()
    nqb, nkb, mt, ws = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64(), ctypes.c_size_t()
    p = pat()
    assert lib.esa_layout_sizes(ctypes.byref(p), ctypes.byref(nqb), ctypes.byref(nkb),
                                ctypes.byref(mt), ctypes.byref(ws)) == en.ESA_OK
    assert (nqb.value, nkb.value) == (256, 256)
    assert mt.value == 32 * sum(qb + 1 for qb in range(256))
    assert mt.value >= 633512
    assert ws.value >= 32 * 256 * 8 * 4 + 32 * 256 * 4
    for bad in [pat(L=0), pat(w=0), pat(nl=0), pat(H=0), pat(bm=0)]:
        assert lib.esa_layout_sizes(ctypes.byref(bad), None, None, None, None) == en.ESA_ERR_SHAPE
    assert lib.esa_layout_sizes(None, None, None, None, None) == en.ESA_ERR_NULL


def test_layout_capacity_bound_holds():
    """The col_idx bound esa_layout_sizes reports covers the real layout."""
    lib = en.load()
    for (L, H, w, nl, layer, bm, bn) in [(1000, 3, 48, 6, 5, 128, 128), (777, 2, 16, 4, 3, 64, 32),
                                         (1024, 4, 64, 8, 7, 128, 128)]:
        p = en.EsaPattern(L, w, layer, nl, H, bm, bn)
        mt = ctypes.c_int64()
        assert lib.esa_layout_sizes(ctypes.byref(p), None, None, ctypes.byref(mt), None) == 0
        idx, msk = elastic_indices(L, layer, nl, H, w)
        rp, _ = block_layout(idx, msk, bm, bn)
        assert int(rp[-1]) <= mt.value


def test_build_entry_points_reject_bad_arguments():
    lib = en.load()
    p = pat(L=1024, H=4)
    fake = ctypes.c_void_p(4096)
    assert lib.esa_build_indices(ctypes.byref(p), 0, 10, fake, fake, 2, None) == en.ESA_ERR_DTYPE
    assert lib.esa_build_indices(ctypes.byref(p), 1000, 100, fake, fake, 8, None) == en.ESA_ERR_SHAPE
    assert lib.esa_build_indices(ctypes.byref(p), 0, 0, fake, fake, 8, None) == en.ESA_OK
    assert lib.esa_build_layout(ctypes.byref(p), None, fake, 1 << 20, fake, 1 << 20, None) == en.ESA_ERR_NULL
    assert lib.esa_build_layout(ctypes.byref(p), fake, fake, 1, fake, 1 << 20, None) == en.ESA_ERR_CAPACITY
    assert lib.esa_build_layout(ctypes.byref(p), fake, fake, 1 << 20, fake, 4, None) == en.ESA_ERR_CAPACITY


def fwd_args(dtype=en.ESA_BF16, B=1, H=4, Hkv=4, Lq=256, Lk=256, D=128, ptr=4096):
    a = en.EsaFwdArgs()
    a.dtype, a.batch, a.num_heads, a.num_kv_heads = dtype, B, H, Hkv
    a.q_len, a.kv_len, a.head_dim = Lq, Lk, D
    a.q = a.k = a.v = a.o = ptr
    for t in "qkvo":
        setattr(a, f"{t}_stride_b", H * Lk * D)
        setattr(a, f"{t}_stride_h", Lk * D)
        setattr(a, f"{t}_stride_s", D)
    a.lse = None
    a.sm_scale = D ** -0.5
    return a


def test_forward_entry_points_reject_bad_arguments():
    lib = en.load()
    p = pat(L=1024, H=4)
    fake = ctypes.c_void_p(4096)
    n = 4 * 2

    # host copy of a 64 x 32 layout's row_ptr (16 query blocks x 4 heads, 3
    # stages each): the stage masks need 192 stages x 64 rows x 1 word
    rp64 = (np.arange(4 * 16 + 1, dtype=np.int32) * 3)
    rph = ctypes.c_void_p(rp64.ctypes.data)

    def call(a, pp=p, items=n, masks=None, words=1 << 20, row_ptr_host=rph):
        return lib.esa_elastic_fwd(ctypes.byref(a), ctypes.byref(pp), fake, fake, row_ptr_host,
                                   masks, words, fake, items, None)

    a = fwd_args()
    a.q = None
    assert call(a) == en.ESA_ERR_NULL
    assert call(fwd_args(dtype=en.ESA_F32)) == en.ESA_ERR_DTYPE
    assert call(fwd_args(dtype=7)) == en.ESA_ERR_DTYPE
    assert call(fwd_args(D=96)) == en.ESA_ERR_UNSUPPORTED
    assert call(fwd_args(Hkv=3)) == en.ESA_ERR_SHAPE
    assert call(fwd_args(Lq=512, Lk=256)) == en.ESA_ERR_SHAPE
    assert call(fwd_args(H=8, Hkv=8)) == en.ESA_ERR_SHAPE  # pattern has 4 heads
    assert call(fwd_args(), items=7) == en.ESA_ERR_SHAPE
    assert call(fwd_args(), items=65) == en.ESA_ERR_SHAPE
    assert call(fwd_args(ptr=4100)) == en.ESA_ERR_ALIGN
    a = fwd_args()
    a.k_stride_s = 130
    assert call(a) == en.ESA_ERR_ALIGN
    # row strides whose span cannot be addressed by 32-bit offsets, including
    # ones whose span overflows int64 (the check must not wrap)
    for big in (1 << 24, 1 << 40, 1 << 62, -(1 << 62)):
        for t in "kv":
            a = fwd_args()
            setattr(a, f"{t}_stride_s", big)
            assert call(a) == en.ESA_ERR_UNSUPPORTED, (t, big)
            assert lib.esa_elastic_fwd_band(ctypes.byref(a), ctypes.byref(p), None, None) \
                == en.ESA_ERR_UNSUPPORTED, (t, big)
    assert call(fwd_args(), pp=pat(L=1024, H=4, bm=64)) == en.ESA_ERR_UNSUPPORTED
    # the band forward takes head dims that are multiples of 8 up to 256
    for bad_d in (100, 264, 4):
        assert lib.esa_elastic_fwd_band(ctypes.byref(fwd_args(D=bad_d)), ctypes.byref(p), None,
                                        None) in (en.ESA_ERR_UNSUPPORTED, en.ESA_ERR_SHAPE), bad_d
    for bad_scale in (0.0, -0.1, float("inf"), float("nan")):
        a = fwd_args()
        a.sm_scale = bad_scale
        assert call(a) == en.ESA_ERR_UNSUPPORTED
    assert call(fwd_args(), pp=pat(L=1024, H=4, layer=9)) == en.ESA_ERR_UNSUPPORTED
    # stage masks: not for 128 x 128 layouts; 8-byte aligned
    assert call(fwd_args(), masks=fake) == en.ESA_ERR_UNSUPPORTED
    assert call(fwd_args(), pp=pat(L=1024, H=4, bm=64, bn=32), items=4 * 16,
                masks=ctypes.c_void_p(4100)) == en.ESA_ERR_ALIGN
    # stage masks are sized on the host from row_ptr_host: a short buffer, or
    # no host row_ptr to size them by, is rejected before any launch
    p64 = pat(L=1024, H=4, bm=64, bn=32)
    words = ctypes.c_int64()
    assert lib.esa_stage_masks_size(ctypes.byref(p64), rph, ctypes.byref(words)) == en.ESA_OK
    assert words.value == 192 * 64
    assert call(fwd_args(), pp=p64, items=4 * 16, masks=fake, words=words.value - 1) \
        == en.ESA_ERR_CAPACITY
    assert call(fwd_args(), pp=p64, items=4 * 16, masks=fake, words=0) == en.ESA_ERR_CAPACITY
    assert call(fwd_args(), pp=p64, items=4 * 16, masks=fake, row_ptr_host=None) \
        == en.ESA_ERR_NULL

    assert lib.esa_elastic_fwd_rows(ctypes.byref(fwd_args(D=258)), ctypes.byref(p), None, None) \
        == en.ESA_ERR_UNSUPPORTED
    assert lib.esa_elastic_fwd_rows(ctypes.byref(fwd_args(Lq=300, Lk=256)), ctypes.byref(p), None,
                                    None) == en.ESA_ERR_SHAPE
    assert lib.esa_sparse_fwd(ctypes.byref(fwd_args()), fake, 2, 0, 0, fake, 1, 0, 0, 64, None) \
        == en.ESA_ERR_DTYPE
    assert lib.esa_sparse_fwd(ctypes.byref(fwd_args()), fake, 8, 0, 0, fake, 2, 0, 0, 64, None) \
        == en.ESA_ERR_DTYPE
    assert lib.esa_sparse_fwd(ctypes.byref(fwd_args()), None, 8, 0, 0, fake, 1, 0, 0, 64, None) \
        == en.ESA_ERR_NULL
    assert lib.esa_sparse_fwd(ctypes.byref(fwd_args()), fake, 8, 0, 0, fake, 1, 0, 0, 0, None) \
        == en.ESA_ERR_SHAPE


def plan(p, row_ptr, q_len, batch):
    lib = en.load()
    n = ctypes.c_int64()
    rp = row_ptr.contiguous()
    st = lib.esa_plan_schedule(ctypes.byref(p), ctypes.c_void_p(rp.data_ptr()), q_len, batch,
                               None, 0, ctypes.byref(n))
    if st != en.ESA_OK:
        return st, None
    items = torch.empty(max(n.value, 1), dtype=torch.int32)
    st = lib.esa_plan_schedule(ctypes.byref(p), ctypes.c_void_p(rp.data_ptr()), q_len, batch,
                               ctypes.c_void_p(items.data_ptr()), n.value, ctypes.byref(n))
    return st, items[:n.value]


@pytest.mark.parametrize("L,Lq,B,H,layer", [(1024, 1024, 1, 4, 4), (1024, 700, 3, 4, 7),
                                            (2048, 2048, 2, 4, 0), (4096, 4096, 1, 32, 4),
                                            (1000, 1000, 1, 1, 3), (300, 100, 1, 2, 5)])
def test_plan_schedule_xcd_runs(L, Lq, B, H, layer):
    """Every item once, -1 pads, 8 interleaved runs (slot % 8) of whole
    streams walked longest block first, with balanced tile counts."""
    w = 64
    p = en.EsaPattern(L, w, layer, 8, H, 128, 128)
    idx, msk = elastic_indices(L, layer, 8, H, w)
    rp, _ = block_layout(idx, msk, 128, 128)
    st, items = plan(p, rp, Lq, B)
    assert st == en.ESA_OK
    nqb = (L + 127) // 128
    nq = (Lq + 127) // 128
    got = items.tolist()
    assert len(got) % 8 == 0 and len(got) <= 8 * B * H * nq
    expect = sorted(((b * H + h) * nqb + qb) for b in range(B) for h in range(H) for qb in range(nq))
    assert sorted(x for x in got if x >= 0) == expect
    assert all(x == -1 or x >= 0 for x in got)

    def cost(it):
        row = (it // nqb) % H * nqb + it % nqb
        return int(rp[row + 1] - rp[row])

    runs = [[x for x in got[r::8]] for r in range(8)]
    flat = []
    for run in runs:
        real = [x for x in run if x >= 0]
        assert run[:len(real)] == real  # pads only at the end of a run
        flat += real
        # within a stream, query blocks descend
        for a, b in zip(real, real[1:]):
            if a // nqb == b // nqb:
                assert a % nqb > b % nqb
    # the runs concatenated walk (batch, head) streams in order
    assert [x // nqb for x in flat] == sorted(x // nqb for x in flat)
    total = sum(cost(x) for x in expect)
    biggest = max(cost(x) for x in expect)
    for run in runs:
        c = sum(cost(x) for x in run if x >= 0)
        assert c <= total / 8 + biggest + 1


@pytest.mark.parametrize("bm,bn", [(64, 32), (128, 64), (128, 128)])
def test_stage_masks_size_and_rejects(bm, bn):
    """Stage-mask words = tiles of the layout x block_m x block_n / 32, from
    the host row_ptr (here the oracle's layout of the same pattern)."""
    lib = en.load()
    L, H, layer = 1000, 3, 5
    p = pat(L=L, H=H, layer=layer, bm=bm, bn=bn)
    idx, msk = elastic_indices(L, layer, 8, H, 64)
    rp, _ = block_layout(idx, msk, bm, bn)
    rph = rp.reshape(-1).to(torch.int32).contiguous()
    assert rph.numel() == H * ((L + bm - 1) // bm) + 1
    words = ctypes.c_int64()
    assert lib.esa_stage_masks_size(ctypes.byref(p), ctypes.c_void_p(rph.data_ptr()),
                                    ctypes.byref(words)) == en.ESA_OK
    assert words.value == int(rph[-1]) * bm * (bn // 32) > 0
    fake = ctypes.c_void_p(4096)
    rpp = ctypes.c_void_p(rph.data_ptr())
    assert lib.esa_build_stage_masks(ctypes.byref(p), fake, fake, rpp, fake, words.value - 1,
                                     None) == en.ESA_ERR_CAPACITY
    assert lib.esa_build_stage_masks(ctypes.byref(p), fake, fake, rpp, ctypes.c_void_p(4100),
                                     words.value, None) == en.ESA_ERR_ALIGN
    assert lib.esa_build_stage_masks(ctypes.byref(p), None, fake, rpp, fake, words.value,
                                     None) == en.ESA_ERR_NULL
    p64 = pat(L=L, H=H, layer=layer, bm=64, bn=64)
    assert lib.esa_stage_masks_size(ctypes.byref(p64), rpp, ctypes.byref(words)) \
        == en.ESA_ERR_UNSUPPORTED


def test_plan_schedule_rejects():
    p = en.EsaPattern(1024, 64, 4, 8, 4, 128, 128)
    rp = torch.zeros(4 * 8 + 1, dtype=torch.int32)
    st, _ = plan(p, rp, 2048, 1)
    assert st == en.ESA_ERR_SHAPE
    lib = en.load()
    n = ctypes.c_int64()
    items = torch.empty(4, dtype=torch.int32)
    assert lib.esa_plan_schedule(ctypes.byref(p), ctypes.c_void_p(rp.data_ptr()), 1024, 1,
                                 ctypes.c_void_p(items.data_ptr()), 4, ctypes.byref(n)) \
        == en.ESA_ERR_CAPACITY
    assert lib.esa_plan_schedule(ctypes.byref(p), None, 1024, 1, None, 0, ctypes.byref(n)) \
        == en.ESA_ERR_NULL


def plan_bwd(p, rp, ci, q_len, batch, hkv):
    lib = en.load()
    nt, ni = ctypes.c_int64(), ctypes.c_int64()
    rp, ci = rp.contiguous(), ci.contiguous()
    vp = ctypes.c_void_p
    st = lib.esa_plan_bwd(ctypes.byref(p), vp(rp.data_ptr()), vp(ci.data_ptr()), q_len, batch, hkv,
                          None, None, None, 0, None, 0, ctypes.byref(nt), ctypes.byref(ni))
    assert st == en.ESA_OK
    nkb = (p.seq_len + 127) // 128
    tile_row = torch.empty(max(int(rp[-1]), 1), dtype=torch.int32)
    kv_ptr = torch.empty(hkv * nkb + 1, dtype=torch.int32)
    kv_tiles = torch.empty(max(nt.value, 1), dtype=torch.int32)
    kv_items = torch.empty(max(ni.value, 1), dtype=torch.int32)
    st = lib.esa_plan_bwd(ctypes.byref(p), vp(rp.data_ptr()), vp(ci.data_ptr()), q_len, batch, hkv,
                          vp(tile_row.data_ptr()), vp(kv_ptr.data_ptr()), vp(kv_tiles.data_ptr()),
                          kv_tiles.numel(), vp(kv_items.data_ptr()), kv_items.numel(),
                          ctypes.byref(nt), ctypes.byref(ni))
    return st, tile_row, kv_ptr, kv_tiles[:nt.value], kv_items[:ni.value]


@pytest.mark.parametrize("L,Lq,B,H,Hkv,layer", [(1024, 1024, 1, 4, 4, 4), (1000, 700, 2, 8, 2, 6),
                                                (2048, 2048, 1, 4, 1, 0), (300, 300, 3, 2, 2, 7)])
def test_plan_bwd_transposes_the_layout(L, Lq, B, H, Hkv, layer):
    """kv lists = for each (kv head, key block), the layout tiles of the group's
    query heads (query blocks below ceil(Lq/128)) holding that key block, in
    (head, query block) order; tile_row inverts the CSR; the kv work list holds
    every (b, kv head, key block) once, in 8 interleaved runs."""
    w = 64
    p = en.EsaPattern(L, w, layer, 8, H, 128, 128)
    idx, msk = elastic_indices(L, layer, 8, H, w)
    rp, ci = block_layout(idx, msk, 128, 128)
    st, tile_row, kv_ptr, kv_tiles, kv_items = plan_bwd(p, rp, ci, Lq, B, Hkv)
    assert st == en.ESA_OK
    nqb = (L + 127) // 128
    nkb = nqb
    nq = (Lq + 127) // 128
    groups = H // Hkv
    for h in range(H):
        for qb in range(nqb):
            for t in range(int(rp[h * nqb + qb]), int(rp[h * nqb + qb + 1])):
                assert int(tile_row[t]) == h * nqb + qb
    for kvh in range(Hkv):
        for kb in range(nkb):
            expect = [t for h in range(kvh * groups, (kvh + 1) * groups) for qb in range(nq)
                      for t in range(int(rp[h * nqb + qb]), int(rp[h * nqb + qb + 1]))
                      if int(ci[t]) == kb]
            r = kvh * nkb + kb
            assert kv_tiles[int(kv_ptr[r]):int(kv_ptr[r + 1])].tolist() == expect
    items = kv_items.tolist()
    assert len(items) % 8 == 0
    assert sorted(x for x in items if x >= 0) == list(range(B * Hkv * nkb))


def test_bwd_entry_points_reject_bad_arguments():
    lib = en.load()
    p = pat(L=1024, H=4)
    fake = ctypes.c_void_p(4096)
    a = en.EsaBwdArgs()
    a.dtype, a.batch, a.num_heads, a.num_kv_heads = en.ESA_BF16, 1, 4, 4
    a.q_len, a.kv_len, a.head_dim = 256, 256, 128
    for name in ("q", "k", "v", "o", "dout", "dq", "dk", "dv"):
        setattr(a, name, 4096)
        setattr(a, f"{name}_stride_b", 4 * 256 * 128)
        setattr(a, f"{name}_stride_h", 256 * 128)
        setattr(a, f"{name}_stride_s", 128)
    a.lse = 4096
    a.lse_stride_b, a.lse_stride_h = 4 * 256, 256
    a.sm_scale = 128 ** -0.5
    ws = ctypes.c_size_t()
    assert lib.esa_bwd_workspace_size(ctypes.byref(a), ctypes.byref(ws)) == en.ESA_OK
    # delta and lse2 (rows padded to 32, + 32), then a flag byte per 16-row
    # dQ group and per 16-key dK / dV block
    assert ws.value == (2 * 1 * 4 * (256 + 32) * 4 + 4 * 16 + 4 * 16 + 255) // 256 * 256

    # host copy of the 128 x 128 layout's row_ptr (8 query blocks x 4 heads,
    # 3 tiles each)
    rp128 = (np.arange(4 * 8 + 1, dtype=np.int32) * 3)
    rph = ctypes.c_void_p(rp128.ctypes.data)
    big = 1 << 24

    def call(args, items=8, kv_items=64, wsb=ws.value, pat_=p, layout=fake, q_list=fake,
             kv_lists=fake, kv_list=fake, masks=fake, q_masks=None, row_ptr_host=rph,
             mask_words=big, q_mask_words=big):
        return lib.esa_elastic_bwd(ctypes.byref(args), ctypes.byref(pat_), layout, layout,
                                   row_ptr_host, q_list, items, kv_lists, kv_lists, kv_lists,
                                   kv_list, kv_items, masks, mask_words, q_masks, q_mask_words,
                                   fake, wsb, None)

    # the block-sparse halves need their layout, lists and masks; the band
    # halves need none of them, and attention_length <= 64
    assert call(a, layout=None) == en.ESA_ERR_NULL
    assert call(a, masks=None) == en.ESA_ERR_NULL
    assert call(a, kv_lists=None) == en.ESA_ERR_NULL
    assert call(a, q_list=None, kv_list=None, layout=None, kv_lists=None, masks=None,
                wsb=16) == en.ESA_ERR_CAPACITY
    assert call(a, q_list=None, kv_list=None, pat_=pat(L=1024, H=4, w=65)) \
        == en.ESA_ERR_UNSUPPORTED
    assert call(a, kv_list=None, kv_items=31, wsb=16) == en.ESA_ERR_CAPACITY  # count ignored
    # row masks serve the block-sparse dQ only, 16-byte aligned
    assert call(a, q_list=None, q_masks=fake) == en.ESA_ERR_UNSUPPORTED
    assert call(a, q_masks=ctypes.c_void_p(4104)) == en.ESA_ERR_ALIGN
    # both mask buffers are sized on the host from row_ptr_host: the key-major
    # masks of the tiles of query blocks 0, 1 of every head (up to the last
    # head's block 1 end, tile 3 * (3 * 8 + 2) = 78) and the row masks of all
    # 96 tiles; shorter buffers, or no host row_ptr, are rejected
    assert call(a, row_ptr_host=None) == en.ESA_ERR_NULL
    assert call(a, q_masks=fake, kv_list=None, masks=None, row_ptr_host=None) == en.ESA_ERR_NULL
    assert call(a, mask_words=78 * 512 - 1) == en.ESA_ERR_CAPACITY
    assert call(a, q_masks=fake, q_mask_words=96 * 128 * 4 - 1) == en.ESA_ERR_CAPACITY
    # (a band dK/dV reads no key-major masks: their size is not checked)
    assert call(a, kv_list=None, masks=None, mask_words=0, items=7) == en.ESA_ERR_SHAPE

    assert call(a, wsb=16) == en.ESA_ERR_CAPACITY
    assert call(a, items=7) == en.ESA_ERR_SHAPE
    assert call(a, kv_items=31) == en.ESA_ERR_SHAPE
    b = en.EsaBwdArgs.from_buffer_copy(a)
    b.dtype = en.ESA_F32
    assert call(b) == en.ESA_ERR_DTYPE
    b = en.EsaBwdArgs.from_buffer_copy(a)
    b.head_dim = 96
    assert call(b) == en.ESA_ERR_UNSUPPORTED
    b = en.EsaBwdArgs.from_buffer_copy(a)
    b.sm_scale = -1.0
    assert call(b) == en.ESA_ERR_UNSUPPORTED
    b = en.EsaBwdArgs.from_buffer_copy(a)
    b.dk = None
    assert call(b) == en.ESA_ERR_NULL
    b = en.EsaBwdArgs.from_buffer_copy(a)
    b.q_len = 300
    assert call(b) == en.ESA_ERR_SHAPE  # q_len > kv_len
    b = en.EsaBwdArgs.from_buffer_copy(a)
    b.dq_stride_s = 130
    assert call(b) == en.ESA_ERR_ALIGN
    # row strides past 32-bit offsets, including spans that overflow int64
    for big in (1 << 24, 1 << 40, 1 << 62):
        for name in ("q", "k", "v", "dout"):
            b = en.EsaBwdArgs.from_buffer_copy(a)
            setattr(b, f"{name}_stride_s", big)
            assert call(b) == en.ESA_ERR_UNSUPPORTED, (name, big)
    # capacity is checked against the tiles of the query blocks q_len covers,
    # read from the host copy of row_ptr
    nqb = (p.seq_len + 127) // 128
    rp_host = (ctypes.c_int32 * (p.num_heads * nqb + 1))(*range(p.num_heads * nqb + 1))
    need = rp_host[(p.num_heads - 1) * nqb + 2]  # q_len = 256: two query blocks
    assert lib.esa_build_tile_masks(ctypes.byref(p), fake, fake, rp_host, 256, fake,
                                    need * 512 - 1, None) == en.ESA_ERR_CAPACITY
    assert lib.esa_build_tile_masks(ctypes.byref(p), fake, fake, None, 256, fake,
                                    need * 512, None) == en.ESA_ERR_NULL
    assert lib.esa_build_tile_masks(ctypes.byref(p), fake, fake, rp_host, 2048, fake, 1 << 30,
                                    None) == en.ESA_ERR_SHAPE


def test_bwd_workspace_size_with_split():
    """Above groups * q_len = 6144 the workspace also holds the band dK/dV's
    split of key block 0: P = ceil(groups * q_len / 6144) (at most 32)
    float32 partial sums of 2 * 16 * D floats and one counter per (batch, kv
    head), after the 2 * B * H * qpad floats of delta and lse2 (each part of
    the workspace 16-byte aligned); then, from the next 256-byte boundary,
    one non-finite flag byte per 16-row dQ group and per 16-key dK / dV
    block, the total a multiple of 256 bytes."""
    lib = en.load()

    def size(B, H, Hkv, q_len, D):
        a = en.EsaBwdArgs()
        a.batch, a.num_heads, a.num_kv_heads, a.q_len, a.kv_len, a.head_dim = B, H, Hkv, q_len, \
            q_len, D
        a.dout_stride_s = D
        ws = ctypes.c_size_t()
        assert lib.esa_bwd_workspace_size(ctypes.byref(a), ctypes.byref(ws)) == en.ESA_OK
        return ws.value

    def expect(B, H, Hkv, q_len, D):
        qpad = (q_len + 31) // 32 * 32 + 32
        n = 2 * B * H * qpad * 4
        parts = min(max(-(-(H // Hkv) * q_len // 6144), 1), 32)
        if parts > 1:
            n += B * Hkv * parts * 2 * 16 * D * 4 + (B * Hkv * 4 + 15) // 16 * 16
        n = (n + 255) // 256 * 256 + B * H * ((q_len + 15) // 16) + B * Hkv * ((q_len + 15) // 16)
        return (n + 255) // 256 * 256

    for shape in [(1, 8, 2, 8192, 128), (2, 4, 4, 6144, 64), (1, 4, 4, 6145, 64),
                  (1, 32, 8, 32768, 128), (1, 64, 1, 131072, 128), (3, 6, 3, 100, 64)]:
        assert size(*shape) == expect(*shape), shape
    # 6144 rows of one group: no split; one more row: two parts
    assert size(1, 1, 1, 6144, 64) == expect(1, 1, 1, 6144, 64) == 2 * (6144 + 32) * 4 + 768


def test_reachability_rejects_bad_arguments():
    lib = en.load()
    f1, f2 = ctypes.c_void_p(4096), ctypes.c_void_p(8192)
    call = lambda L, w, nl, H, pos, r=f1, wk=f2, c=None: lib.esa_reachability(L, w, nl, H, pos, r,
                                                                            wk, c, None)
    assert call(1024, 64, 8, 8, 1024) == en.ESA_ERR_SHAPE   # position == seq_len
    assert call(1024, 64, 8, 8, -1) == en.ESA_ERR_SHAPE
    assert call(1024, 0, 8, 8, 10) == en.ESA_ERR_SHAPE      # attn_length <= 0
    assert call(1024, 64, 0, 8, 10) == en.ESA_ERR_SHAPE     # no layers
    assert call(1024, 64, 8, 0, 10) == en.ESA_ERR_SHAPE     # no heads
    assert call(1024, 64, 8, 8, 10, r=None) == en.ESA_ERR_NULL
    assert call(1024, 64, 8, 8, 10, wk=None) == en.ESA_ERR_NULL
    assert call(1024, 64, 8, 8, 10, wk=f1) == en.ESA_ERR_SHAPE   # reach and work alias
    assert call(1024, 64, 8, 8, 10, c=ctypes.c_void_p(4098)) == en.ESA_ERR_ALIGN


def test_hole_checker_validates_before_the_gpu():
    import check_attn_hole as ch
    with pytest.raises(ValueError, match="position_id must be between 0 and 99"):
        ch.attention_reachability(100, 8, 8, 64, position_id=100)
    with pytest.raises(ValueError, match="attn_length must be positive"):
        ch.attention_reachability(100, 8, 8, 0)


def test_noalloc_rejects_oversized_workspace():
    """esa_elastic_bwd_noalloc refuses a backward whose workspace would
    exceed its per-device array before any HIP call (ESA_ERR_CAPACITY)."""
    lib = en.load()
    cap = lib.esa_bwd_noalloc_max_workspace()
    a = en.EsaBwdArgs()
    a.dtype = en.ESA_BF16
    a.batch, a.num_heads, a.num_kv_heads, a.q_len, a.kv_len, a.head_dim = 8, 32, 32, 32768, 32768, 128
    need = ctypes.c_size_t()
    assert lib.esa_bwd_workspace_size(ctypes.byref(a), ctypes.byref(need)) == en.ESA_OK
    assert need.value > cap
    fake = 1 << 20
    for name in ("q", "k", "v", "o", "dout", "dq", "dk", "dv", "lse"):
        setattr(a, name, fake)
    a.q_stride_b, a.q_stride_h, a.q_stride_s = 32 * 32768 * 128, 32768 * 128, 128
    for name in ("k", "v", "dq", "dk", "dv"):
        setattr(a, f"{name}_stride_b", a.q_stride_b)
        setattr(a, f"{name}_stride_h", a.q_stride_h)
        setattr(a, f"{name}_stride_s", a.q_stride_s)
    for name in ("o", "dout"):
        setattr(a, f"{name}_stride_b", 32768 * 32 * 128)
        setattr(a, f"{name}_stride_h", 128)
        setattr(a, f"{name}_stride_s", 32 * 128)
    a.lse_stride_b, a.lse_stride_h = 32 * 32768, 32768
    a.sm_scale = 128 ** -0.5
    p = en.EsaPattern(32768, 64, 4, 8, 32, 128, 128)
    st = lib.esa_elastic_bwd_noalloc(ctypes.byref(a), ctypes.byref(p), None, None, None, None, 0,
                                     None, None, None, None, 0, None, 0, None, 0, None)
    assert st == en.ESA_ERR_CAPACITY


def bwd_args(dtype=en.ESA_F32, B=2, H=4, Hkv=2, Lq=100, Lk=120, D=64, ptr=1 << 20):
    a = en.EsaBwdArgs()
    a.dtype, a.batch, a.num_heads, a.num_kv_heads = dtype, B, H, Hkv
    a.q_len, a.kv_len, a.head_dim = Lq, Lk, D
    for name in ("q", "o", "dout", "dq"):
        setattr(a, name, ptr)
        setattr(a, f"{name}_stride_b", H * Lq * D)
        setattr(a, f"{name}_stride_h", Lq * D)
        setattr(a, f"{name}_stride_s", D)
    for name in ("k", "v", "dk", "dv"):
        setattr(a, name, ptr)
        setattr(a, f"{name}_stride_b", Hkv * Lk * D)
        setattr(a, f"{name}_stride_h", Lk * D)
        setattr(a, f"{name}_stride_s", D)
    a.lse = ptr
    a.lse_stride_b, a.lse_stride_h = H * Lq, Lq
    a.sm_scale = D ** -0.5
    return a


def test_gather_bwd_workspace_size_host_only():
    """The gather backward's workspace is a host-side formula (no device
    query): per batch element and entry two float32 coefficients, four uint32
    arrays of entries for the sort, Hkv * kv_len + 1 segment starts, and the
    sort's per-tile digit histograms (256 per 4096 entries, twice) and their
    scan's chunk sums, each region rounded up to 256 bytes."""
    lib = en.load()
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    for (B, H, Hkv, Lq, Lk, w) in [(2, 4, 2, 100, 120, 24), (1, 32, 8, 32768, 32768, 64),
                                   (3, 1, 1, 1, 5, 1)]:
        a = bwd_args(B=B, H=H, Hkv=Hkv, Lq=Lq, Lk=Lk)
        ws = ctypes.c_size_t()
        assert lib.esa_gather_bwd_workspace_size(ctypes.byref(a), w, ctypes.byref(ws)) == 0
        E = H * Lq * w
        nb = (E + 4095) // 4096
        want = (2 * up(B * E * 4) + 4 * up(E * 4) + up((Hkv * Lk + 1) * 4) +
                2 * up(256 * nb * 4) + up((256 * nb + 2047) // 2048 * 4))
        assert ws.value == want
    a = bwd_args(H=32, Lq=1 << 20)
    assert lib.esa_gather_bwd_workspace_size(ctypes.byref(a), 128, ctypes.byref(ws)) \
        == en.ESA_ERR_SHAPE  # entry ids would pass 2^31


def test_gather_entry_points_reject_bad_arguments():
    lib = en.load()
    fake = ctypes.c_void_p(1 << 20)
    ws_need = ctypes.c_size_t()
    a = bwd_args()
    assert lib.esa_gather_bwd_workspace_size(ctypes.byref(a), 24, ctypes.byref(ws_need)) == 0

    def sparse(b, w=24, ws=ws_need.value, ib=8, mb=8):
        return lib.esa_sparse_bwd(ctypes.byref(b), fake, ib, 100 * w, w, fake, mb, 100 * w, w, w,
                                  fake, ws, None)

    assert sparse(a, ws=ws_need.value - 1) == en.ESA_ERR_CAPACITY
    assert sparse(a, ib=2) == en.ESA_ERR_DTYPE
    assert sparse(a, mb=2) == en.ESA_ERR_DTYPE
    assert sparse(bwd_args(dtype=9)) == en.ESA_ERR_DTYPE
    assert sparse(bwd_args(D=66)) == en.ESA_ERR_UNSUPPORTED
    assert sparse(bwd_args(D=260)) == en.ESA_ERR_UNSUPPORTED
    assert sparse(bwd_args(Hkv=3)) == en.ESA_ERR_SHAPE
    b = bwd_args()
    b.dk = None
    assert sparse(b) == en.ESA_ERR_NULL
    b = bwd_args(dtype=en.ESA_BF16)
    b.k_stride_s = 66
    assert sparse(b) == en.ESA_ERR_ALIGN
    assert lib.esa_sparse_bwd(ctypes.byref(a), None, 8, 0, 0, fake, 8, 0, 0, 24, fake,
                              ws_need.value, None) == en.ESA_ERR_NULL
    # the pattern path
    p = pat(L=1024, H=4, w=24)
    assert lib.esa_elastic_bwd_rows(ctypes.byref(a), ctypes.byref(p), None, 1.0, 0, fake,
                                    ws_need.value, None) == en.ESA_ERR_SHAPE  # dropout_p = 1
    assert lib.esa_elastic_bwd_rows(ctypes.byref(a), ctypes.byref(pat(L=1024, H=8, w=24)), None,
                                    0.0, 0, fake, ws_need.value, None) == en.ESA_ERR_SHAPE
    assert lib.esa_elastic_bwd_rows(ctypes.byref(a), ctypes.byref(p), None, 0.0, 0, None,
                                    ws_need.value, None) == en.ESA_ERR_NULL
    # the naive forward
    f = fwd_args(dtype=en.ESA_F16, H=4, Hkv=4)
    opts = en.EsaNaiveOpts()
    opts.dropout_p = 1.5
    assert lib.esa_elastic_fwd_naive(ctypes.byref(f), ctypes.byref(pat(L=1024, H=4)), None,
                                     ctypes.byref(opts), None) == en.ESA_ERR_SHAPE
    opts.dropout_p = 0.1
    opts.weights = 1 << 20
    assert lib.esa_elastic_fwd_naive(ctypes.byref(f), ctypes.byref(pat(L=1024, H=4)), None,
                                     ctypes.byref(opts), None) == en.ESA_ERR_NULL  # no lse
    assert lib.esa_elastic_fwd_naive(ctypes.byref(f), ctypes.byref(pat(L=1024, H=4)), None,
                                     None, None) == en.ESA_ERR_NULL
