"""The rate probes of libesa_probe.so (GPU): each writes a closed form of its
inputs per thread, which pins that the work the rate is computed from was
done (bench.py --peaks times them)."""
import ctypes

import pytest
import torch

import esa_native as en

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)


def test_mfma_probe_closed_form():
    lib = en.load_probe()
    wg, iters = 64, 100
    sink = torch.full((wg * 256,), -1.0, dtype=torch.float32, device=DEV)
    en.check(lib.esa_probe_mfma_bf16(wg, iters, 0x3f80, ctypes.c_void_p(sink.data_ptr()),
                                     sink.numel(), _stream()), "esa_probe_mfma_bf16")
    torch.cuda.synchronize()
    # 4 chains x 16 accumulators per lane, each + 16 per MFMA (1.0 x 1.0 over k = 16)
    assert torch.all(sink == 64.0 * 16 * iters)


def test_l2_to_lds_probe_closed_form():
    lib = en.load_probe()
    wg, iters, region = 48, 37, 16384 * 5
    src = torch.full((region // 2,), 3, dtype=torch.int16, device=DEV)
    sink = torch.zeros(wg * 256, dtype=torch.int32, device=DEV)
    for stride in (7, iters):
        sink.zero_()
        en.check(lib.esa_probe_l2_to_lds(ctypes.c_void_p(src.data_ptr()), region, wg, iters,
                                         stride, ctypes.c_void_p(sink.data_ptr()), sink.numel(),
                                         _stream()), "esa_probe_l2_to_lds")
        torch.cuda.synchronize()
        assert torch.all(sink == 8 * 3)


def test_hbm_read_probe_closed_form():
    lib = en.load_probe()
    wg, n = 40, (1 << 20) + 48  # words: not a multiple of the grid, tail loop taken
    src = torch.arange(n, dtype=torch.int32, device=DEV)
    sink = torch.zeros(wg * 256, dtype=torch.int32, device=DEV)
    en.check(lib.esa_probe_hbm_read(ctypes.c_void_p(src.data_ptr()), n * 4, wg,
                                    ctypes.c_void_p(sink.data_ptr()), sink.numel(), _stream()),
             "esa_probe_hbm_read")
    torch.cuda.synchronize()
    total = int(sink.to(torch.int64).sum().item()) % (1 << 32)
    assert total == (n * (n - 1) // 2) % (1 << 32)


def test_gather_probe_closed_form():
    lib = en.load_probe()
    wg, src_rows, n = 24, 5000, 20011  # a ragged last round
    src = torch.arange(src_rows * 64, dtype=torch.int32, device=DEV)  # 256-byte rows
    g = torch.Generator(device="cpu").manual_seed(5)
    rows = torch.randint(-3, src_rows + 3, (n,), generator=g, dtype=torch.int32)  # some clamped
    rows_d = rows.to(DEV)
    sink = torch.zeros(wg * 256, dtype=torch.int32, device=DEV)
    en.check(lib.esa_probe_gather_read(ctypes.c_void_p(src.data_ptr()), src_rows,
                                       ctypes.c_void_p(rows_d.data_ptr()), n, wg,
                                       ctypes.c_void_p(sink.data_ptr()), sink.numel(), _stream()),
             "esa_probe_gather_read")
    torch.cuda.synchronize()
    r = rows.clamp(0, src_rows - 1).to(torch.int64)
    want = int((r * 64 * 64 + 63 * 64 // 2).sum().item()) % (1 << 32)  # sum of row r's words
    assert int(sink.to(torch.int64).sum().item()) % (1 << 32) == want


def test_gather_to_lds_probe_closed_form():
    lib = en.load_probe()
    wg, iters, src_rows, n = 40, 9, 777, 64 * 13
    src = torch.full((src_rows * 128,), 5, dtype=torch.int16, device=DEV)
    g = torch.Generator(device="cpu").manual_seed(6)
    rows = torch.randint(-2, src_rows + 2, (n,), generator=g, dtype=torch.int32).to(DEV)
    sink = torch.zeros(wg * 256, dtype=torch.int32, device=DEV)
    en.check(lib.esa_probe_gather_to_lds(ctypes.c_void_p(src.data_ptr()), src_rows,
                                         ctypes.c_void_p(rows.data_ptr()), n, wg, iters,
                                         ctypes.c_void_p(sink.data_ptr()), sink.numel(),
                                         _stream()), "esa_probe_gather_to_lds")
    torch.cuda.synchronize()
    assert torch.all(sink == 8 * 5)


@pytest.mark.parametrize("pattern", [0, 1, 2, 3])
def test_lds_read_probe_closed_form(pattern):
    """Every read of every pattern lands in the wave's slot of 16-bit ones:
    32 words per round per thread (four 16-byte or eight 8-byte reads)."""
    lib = en.load_probe()
    wg, iters = 24, 37
    sink = torch.zeros(wg * 256, dtype=torch.int32, device=DEV)
    en.check(lib.esa_probe_lds_read(pattern, wg, iters, ctypes.c_void_p(sink.data_ptr()),
                                    sink.numel(), _stream()), "esa_probe_lds_read")
    torch.cuda.synchronize()
    assert torch.all(sink == 32 * iters)
