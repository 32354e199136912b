"""Benchmark: elastic block-sparse attention forward on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config 32k|8k|batched|128k]
                    [--layer N] [--no-cpu] [--no-backward] [--no-decode]
                    [--no-configs] [--no-chunk]
    python bench.py --peaks            (only the rate probes, one JSON line)
    python bench.py --lds-probe        (only the LDS operand-read probes)

A step is one ElasticSparseAttention.forward over one batch of synthetic
input already resident in HBM (the module's drop-in HIP path: one kernel
launch, the band-gathered kernel or the block-sparse tile kernel, whichever
is faster for the shape; config.kernel names it).  The block layout is built
before the timed region, as the reference builds its index cache at
construction; its build time is reported separately.

Prints ONE JSON line.

value            the metric: counted active-tile flops / wall time per step,
                 counted flops = active 128x128 tiles x 4 * 128 * 128 * D
                 (the metric's unit of work, whatever the kernel executes);
                 counted_pct_of_bf16_peak is value / 2.5 PFLOP/s.  This is
                 not an MFMA utilisation: the kernels skip most of those
                 flops.
roofline         the timed kernel against the resource it uses, from the work
                 it executes: at dilated layers its issued bf16 MFMA flops
                 (the tile kernel: the 32 x 32 blocks of active tiles that
                 hold a valid key for a row of the wave; the band kernel: 16
                 keys x 16 rows per index-list entry pair, equal to the
                 profiled SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512) over its mean
                 launch time (HIP events on the launch stream), against 2.5
                 PFLOP/s; at layer 0 (a sliding window, ~127 flop/B) the
                 algorithmic bytes over that time against 8 TB/s.  traffic =
                 profiled HBM bytes per launch (FETCH_SIZE and WRITE_SIZE
                 scaled by a plain copy's readings), from the committed
                 summary in profiles/, else null.
l2_to_cu         what bounds the kernels at dilated layers: bytes gathered
                 from L2 (profiled) over the kernel time, against the L2 ->
                 LDS rates measured in the same run by the rate probes
                 (256-byte rows at random positions of an L2-resident region,
                 the band kernels' pattern, as the ceiling; 16 KB streaming
                 rounds beside it).
configs          every configured workload (forward and backward kernel
                 times, kernel-only, a few steps each) at layers 0, 4 and 7.
backward         the backward of the headline forward (dQ, dK, dV).
decode           one decode step of 128 sequences through the module's
                 cache_position path.
chunked_prefill  the headline's last 4096 rows as a cache_position chunk
                 through the module (the band kernel at those positions),
                 beside the same rows' share of the full prefill.
cpu_baseline     the reference's PyTorch fallback (_naive_forward, restated
                 in oracle/) on the host cores over every third 256-row chunk
                 of the headline forward, median of three runs, scaled to the
                 whole forward (about 8 s a run).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "elastic-sparse-attention_amd"))

CONFIGS = {
    # name: (B, H, L, D, input scale, outlier fraction)
    "32k": (1, 32, 32768, 128, 128 ** -0.25, 0.0),
    "8k": (1, 32, 8192, 128, 128 ** -0.25, 0.0),
    "batched": (8, 16, 4096, 64, 1.0, 0.0),
    "128k": (1, 8, 131072, 128, 1.0, 0.01),
}
# the configs object: every configured workload at these layers (the
# headline's own layer is the main line)
CONFIG_LAYERS = {"8k": (0, 4, 7), "batched": (0, 4, 7), "128k": (0, 4, 7), "32k": (0, 7)}
W, NL = 64, 8
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
METRIC = "active-block TFLOP/s + % of bf16 MFMA peak, elastic attn fwd, 1 GPU, L=32K"


def host_cores() -> int:
    """Cores this process may run on (its CPU affinity set)."""
    return len(os.sched_getaffinity(0))


def cpu_baseline(cfg_name: str, layer: int, counted_flops: float, chunk_rows: int = 256,
                 every: int = 3, runs: int = 3) -> dict:
    """The reference's PyTorch fallback on the host over a bounded sample of
    the whole forward: every ``every``-th chunk of ``chunk_rows`` query rows
    (spread over the sequence, all heads), timed ``runs`` times after a
    one-chunk warm-up; the median run, scaled by all rows / sampled rows,
    gives the whole forward's time (a row's cost does not depend on its
    position: it gathers the same ``w`` keys)."""
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from esa_oracle import elastic_indices, naive_forward, seeded_inputs

    B, H, L, D, scale, outl = CONFIGS[cfg_name]
    cores = host_cores()
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = min(cores, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else cores
    torch.set_num_threads(threads)
    q, k, v = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=0, scale=scale,
                            outlier_frac=outl)
    t0 = time.perf_counter()
    idx, msk = elastic_indices(L, layer, NL, H, W)
    layout_s = time.perf_counter() - t0
    starts = list(range(0, L, chunk_rows * every))
    rows = sum(min(chunk_rows, L - c0) for c0 in starts)

    def sample() -> None:
        for c0 in starts:
            c1 = min(c0 + chunk_rows, L)
            naive_forward(q[:, :, c0:c1], k, v, idx, msk, D ** -0.5, 1, L,
                          cache_position=torch.arange(c0, c1), chunk_rows=chunk_rows)

    naive_forward(q[:, :, :chunk_rows], k, v, idx, msk, D ** -0.5, 1, L,
                  cache_position=torch.arange(chunk_rows), chunk_rows=chunk_rows)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        sample()
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    full_s = med * L / rows
    return {"value": counted_flops / full_s / 1e12, "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": (f"reference PyTorch fallback (_naive_forward restated, bf16), B={B}, "
                       f"{H} heads, layer {layer}: one {chunk_rows}-row chunk in every {every} "
                       f"of the {L} query rows ({rows} rows), median of {runs} runs after a "
                       f"one-chunk warm-up = {med:.2f} s (runs "
                       + ", ".join(f"{t:.2f}" for t in times) +
                       f" s), scaled by {L}/{rows} to the whole forward; {threads} threads "
                       f"of {cores} cores in the affinity set"),
            "seconds_per_forward": round(full_s, 3), "sample_runs_s": [round(t, 3) for t in times],
            "layout_build_s": round(layout_s, 4)}


COPY_BYTES = 1 << 30


def copy_calibration(torch) -> None:
    """A plain device-to-device copy of COPY_BYTES, three times: the kernel
    whose FETCH_SIZE / WRITE_SIZE readings scale the counters to bytes."""
    dev = torch.device("cuda", 0)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "copies": 3}), flush=True)


def l2_lds_rates(torch, lib, steps: int, pers=(2, 5, 8)) -> dict:
    """L2 -> LDS through buffer_load ... lds, best over `pers` workgroups per
    CU, each the median of `steps` timed launches with its result checked:
    16 KB rounds from a 1 MiB region every XCD's L2 holds ("stream"), and
    256-byte rows at random positions of the same region, four per DMA
    instruction ("gather", the band kernels' pattern).  TB/s, with the
    sweeps."""
    import ctypes
    import esa_native as en
    dev = torch.device("cuda", 0)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    vp = ctypes.c_void_p
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    region = 1 << 20
    src = torch.full((region // 2,), 1, dtype=torch.int16, device=dev)
    n = 1 << 20
    g = torch.Generator(device=dev).manual_seed(12)
    rows = torch.randint(0, region // 256, (n,), generator=g, device=dev, dtype=torch.int32)
    out = {}
    for name in ("stream", "gather"):
        rates = {}
        for per in pers:
            wg, iters = per * cus, 2048 // per
            sink = torch.empty(wg * 256, dtype=torch.int32, device=dev)
            if name == "stream":
                call = lambda: en.check(lib.esa_probe_l2_to_lds(  # noqa: E731
                    vp(src.data_ptr()), region, wg, iters, 7, vp(sink.data_ptr()), sink.numel(),
                    stream), "l2 probe")
            else:
                call = lambda: en.check(lib.esa_probe_gather_to_lds(  # noqa: E731
                    vp(src.data_ptr()), region // 256, vp(rows.data_ptr()), n, wg, iters,
                    vp(sink.data_ptr()), sink.numel(), stream), "l2 gather probe")
            ms = event_ms(torch, call, steps, 3)
            assert bool(torch.all(sink == 8)), f"l2 {name} probe result"
            rates[per] = wg * iters * 16384 / (ms * 1e-3) / 1e12
            del sink
        per, tbs = max(rates.items(), key=lambda kv: kv[1])
        out[name] = {"tbs": round(tbs, 2), "workgroups_per_cu": per,
                     "sweep": {str(k): round(v, 3) for k, v in rates.items()}}
    return out


LDS_PATTERNS = {0: "K operand ds_read_b128, kernels' swizzle",
                1: "V^T operand ds_read_b64_tr_b16, kernels' swizzle",
                2: "ds_read_b64_tr_b16, contiguous 16-dim slices, 8 bank groups per 16 lanes",
                3: "K operand ds_read_b128, unswizzled"}


def lds_probe(torch, steps: int = 10) -> dict:
    """The band forward's LDS operand reads at D = 128 (esa_probe_lds_read),
    each pattern the median of `steps` timed launches of 2 workgroups (8
    waves) per CU, its result checked: ns per wave-level LDS instruction per
    CU.  Bank-conflict cycles per instruction come from a counter run
    (rocprofv3 --pmc SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT) of this command."""
    import ctypes
    import esa_native as en
    lib = en.load_probe()
    dev = torch.device("cuda", 0)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    wg, iters = 2 * cus, 4096
    sink = torch.empty(wg * 256, dtype=torch.int32, device=dev)
    out = {}
    for pat, desc in LDS_PATTERNS.items():
        ms = event_ms(torch, lambda: en.check(lib.esa_probe_lds_read(
            pat, wg, iters, ctypes.c_void_p(sink.data_ptr()), sink.numel(), stream),
            "lds probe"), steps, 3)
        assert bool(torch.all(sink == 32 * iters)), "lds probe result"
        per_wave = iters * (4 if pat in (0, 3) else 8)
        out[str(pat)] = {"pattern": desc,
                         "ns_per_instr_per_cu": round(ms * 1e6 / (wg * 4 * per_wave / cus), 3)}
    return out


def peaks(torch, steps: int = 10) -> None:
    """The rates the roofline is stated against, measured on this GPU with
    libesa_probe.so (include/esa_probe.h), each the median of `steps` timed
    launches after warm-ups, with its closed-form result checked, and the
    best over a few launch shapes (workgroups per CU) reported with its
    shape: dense bf16 MFMA (four independent 32x32x16 chains per wave), HBM
    read (a 4 GiB buffer streamed once), a device copy (1 GiB, read +
    write), and L2 -> LDS through buffer_load ... lds (a 1 MiB region every
    XCD's L2 holds, 16 KB rounds per workgroup, two in flight) and HBM ->
    LDS through the same path (a 2 GiB region read once), 256-byte rows at
    random positions of the L2-resident region into LDS (the band kernels'
    pattern), and 256-byte row gathers at random positions of HBM into
    registers (the decode step's)."""
    import ctypes
    import esa_native as en
    lib = en.load_probe()
    dev = torch.device("cuda", 0)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    vp = ctypes.c_void_p
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    out = {"cus": cus}

    def best(rates):
        per, rate = max(rates.items(), key=lambda kv: kv[1])
        return per, rate, {str(k): round(v, 3) for k, v in rates.items()}

    rates = {}
    for per in (2, 4):
        wg, iters = per * cus, 32768 // per
        sink = torch.empty(wg * 256, dtype=torch.float32, device=dev)
        ms = event_ms(torch, lambda: en.check(lib.esa_probe_mfma_bf16(
            wg, iters, 0x3f80, vp(sink.data_ptr()), sink.numel(), stream), "mfma probe"),
            steps, 3)
        assert bool(torch.all(sink == 64.0 * 16 * iters)), "mfma probe result"
        rates[per] = wg * 4 * iters * 4 * 32768 / (ms * 1e-3) / 1e12
        del sink
    per, tf, sweep = best(rates)
    out["mfma_bf16"] = {"tflops": round(tf, 1), "workgroups_per_cu": per, "sweep": sweep,
                        "published": PEAK_BF16_TFLOPS,
                        "frac_of_published": round(tf / PEAK_BF16_TFLOPS, 4)}

    nbytes = 4 << 30
    src = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    rates = {}
    for per in (1, 2, 3, 4, 32):
        wg = per * cus
        sink = torch.empty(wg * 256, dtype=torch.int32, device=dev)
        ms = event_ms(torch, lambda: en.check(lib.esa_probe_hbm_read(
            vp(src.data_ptr()), nbytes, wg, vp(sink.data_ptr()), sink.numel(), stream),
            "hbm probe"), steps, 3)
        assert int(sink.to(torch.int64).sum().item()) % (1 << 32) == \
            (nbytes // 4) % (1 << 32), "hbm probe result"
        rates[per] = nbytes / (ms * 1e-3) / 1e12
        del sink
    per, tbs, sweep = best(rates)
    out["hbm_read"] = {"tbs": round(tbs, 3), "workgroups_per_cu": per, "sweep": sweep,
                       "published": PEAK_HBM_GBS / 1e3,
                       "frac_of_published": round(tbs * 1e3 / PEAK_HBM_GBS, 4)}
    del src

    a = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    ms = event_ms(torch, lambda: b.copy_(a), steps, 3)
    out["copy"] = {"tbs_read_plus_write": round(2 * COPY_BYTES / (ms * 1e-3) / 1e12, 3)}
    del a, b

    l2 = l2_lds_rates(torch, lib, steps)
    out["l2_to_lds"] = l2["stream"]
    out["l2_gather_256b_to_lds"] = l2["gather"]

    # the same DMA path from HBM: a 2 GiB region, each chunk read once
    region = (1 << 31) - 16384
    src = torch.full((region // 2,), 1, dtype=torch.int16, device=dev)
    rates = {}
    for per in (2, 4, 8):
        wg = per * cus
        iters = region // 16384 // wg
        sink = torch.empty(wg * 256, dtype=torch.int32, device=dev)
        ms = event_ms(torch, lambda: en.check(lib.esa_probe_l2_to_lds(
            vp(src.data_ptr()), region, wg, iters, iters, vp(sink.data_ptr()), sink.numel(),
            stream), "hbm -> lds probe"), steps, 3)
        assert bool(torch.all(sink == 8)), "hbm -> lds probe result"
        rates[per] = wg * iters * 16384 / (ms * 1e-3) / 1e12
        del sink
    per, tbs, sweep = best(rates)
    out["hbm_to_lds"] = {"tbs": round(tbs, 3), "workgroups_per_cu": per, "sweep": sweep}
    del src

    # 256-byte row gathers at random positions of a 4 GiB region (the decode
    # step's access pattern: 524288 rows, as B=128 x H=32 x 64 K and V rows)
    src_rows = (4 << 30) // 256
    src = torch.ones(src_rows * 64, dtype=torch.int32, device=dev)
    n = 128 * 32 * 64 * 2
    g = torch.Generator(device=dev).manual_seed(11)
    rows = torch.randint(0, src_rows, (n,), generator=g, device=dev, dtype=torch.int32)
    rates = {}
    for per in (2, 4, 8):
        wg = per * cus
        sink = torch.empty(wg * 256, dtype=torch.int32, device=dev)
        ms = event_ms(torch, lambda: en.check(lib.esa_probe_gather_read(
            vp(src.data_ptr()), src_rows, vp(rows.data_ptr()), n, wg, vp(sink.data_ptr()),
            sink.numel(), stream), "gather probe"), steps, 3)
        assert int(sink.to(torch.int64).sum().item()) % (1 << 32) == (n * 64) % (1 << 32), \
            "gather probe result"
        rates[per] = n * 256 / (ms * 1e-3) / 1e12
        del sink
    per, tbs, sweep = best(rates)
    out["hbm_gather_256b"] = {"tbs": round(tbs, 3), "workgroups_per_cu": per, "sweep": sweep,
                              "rows": n}
    out["lds_read"] = lds_probe(torch, steps)
    print(json.dumps({"peaks": out}), flush=True)


WARM_MS = 50.0  # the GPU's clocks climb over tens of ms of work after idle time


def event_ms(torch, fn, steps: int, warmup: int) -> float:
    """Median time of `fn` over `steps` calls after `warmup` untimed ones (and
    more until WARM_MS of them have run), each between two HIP events on
    torch's current stream (the stream the library launches on)."""
    t0 = time.perf_counter()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    while (time.perf_counter() - t0) * 1e3 < WARM_MS:
        for _ in range(max(warmup, 1)):
            fn()
        torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    torch.cuda.synchronize()
    for s_ev, e_ev in evs:
        s_ev.record(stream)
        fn()
        e_ev.record(stream)
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in evs)


def executed_blocks(torch, lay, L: int) -> int:
    """Number of (active tile, 32-row block, 32-key block) triples in which
    some row has a valid key, per batch element, over the query blocks of
    an L-row prefill: the blocks the tile forward issues MFMAs for.  From
    the layout's key-major tile masks (32 row bits per key)."""
    masks = lay.tile_masks(L)
    n = lay.mask_tiles(L)
    H, nqb = lay.pattern.num_heads, lay.num_qblocks
    rp = lay.row_ptr_host.to(torch.int64)
    # the mask buffer holds the tiles of every query block of the heads
    # before the last: keep those of the blocks below ceil(L / block_m)
    tile_qb = torch.repeat_interleave(torch.arange(H * nqb) % nqb, rp[1:] - rp[:-1])[:n]
    keep = (tile_qb < (L + lay.pattern.block_m - 1) // lay.pattern.block_m).to(masks.device)
    blocks = masks[:n * 512].view(n, 4, 4, 32).ne(0).any(-1)
    return int(blocks[keep].sum().item())


def band_executed_flops(B: int, H: int, L: int, D: int, w: int) -> float:
    """MFMA flops the band kernel issues in its main loop: per 16-row group
    and pair of index-list entries with a valid key in the group, D/32 QK^T
    and D/16 PV 16x16x32 MFMAs per entry pair (2 D/32 + D/16 in all), 16384
    flops each.  Entries j > i are masked for rows i < w - 1, so group g
    holds min(w, 16 g + 16) live entries."""
    pairs = 0
    for g in range((L + 15) // 16):
        live = min(w, 16 * g + 16)
        pairs += (live + 1) // 2
    return float(B * H * pairs * (2 * (D // 32) + D // 16) * 16384)


def window_executed_flops(B: int, H: int, L: int, D: int, w: int, G: int = 2) -> float:
    """MFMA flops the window kernel (the band entry point at interpolation
    weight 0) issues: per 16 G-row group, its keys [max(r0 - w + 1, 0),
    min(r0 + 16 G, L)) in pairs of 16-key chunks, and per pair and 16-row
    group 2 D/32 QK^T MFMAs (one per chunk) and D/16 PV MFMAs (the pair as
    one 32-key step), 16384 flops each."""
    pairs = 0
    for r0 in range(0, L, 16 * G):
        pairs += (min(r0 + 16 * G, L) - max(r0 - w + 1, 0) + 31) // 32
    return float(B * H * pairs * G * (2 * (D // 32) + D // 16) * 16384)


def band_bwd_executed_flops(torch, lay, B: int, H: int, Hkv: int, L: int, D: int,
                            w: int) -> dict:
    """MFMA flops the band backward kernels issue in their main loops
    (16x16x32 MFMAs, 16384 flops each; wide-band tail passes left out):
    band_dq_kernel per 16-row group and entry pair with a valid key in the
    group, 2 D/32 for S^T, 2 D/32 for dP^T and D/16 for dQ^T; band_dkdv_kernel
    per 16-key block, query head of its kv group and 32-row step of the
    (row, entry) pairs whose key lies in the block (ceil(pairs / 32) steps),
    2 D/32 for S, 2 D/32 for dP, D/16 each for dV^T and dK^T.  The pairs per
    (head, block) are counted from the pattern's index lists built on the
    GPU.  At layer 0 (interpolation weight 0, a sliding window) the kernels
    walk the window directly: window_dq_kernel per 32-row group and pair of
    16-key chunks of keys [max(32 g - w + 1, 0), min(32 g + 32, L)), the
    MFMAs of a pair for each of the group's two 16-row halves;
    band_dkdv_kernel per block, query head and 32-row step of rows
    [16 b, min(16 b + 15 + w, L)), with the same MFMAs per step."""
    from elastic_sparse_attention import build_indices
    dq_unit = (4 * (D // 32) + D // 16) * 16384
    dkdv_unit = (4 * (D // 32) + 2 * (D // 16)) * 16384
    if lay.pattern.layer_idx == 0:
        pairs = steps = 0
        for g in range((L + 31) // 32):
            pairs += 2 * ((min(32 * g + 32, L) - max(32 * g - w + 1, 0) + 31) // 32)
        for g in range((L + 15) // 16):
            steps += (min(16 * g + 15 + w, L) - 16 * g + 31) // 32
        return {"dq": float(B * H * pairs * dq_unit), "dkdv": float(B * H * steps * dkdv_unit)}
    pairs = 0
    for g in range((L + 15) // 16):
        pairs += (min(w, 16 * g + 16) + 1) // 2
    dq = float(B * H * pairs * dq_unit)
    idx, msk = build_indices(lay.pattern, lay.device, torch.int32)
    nblk = (L + 15) // 16
    steps = 0
    for h in range(H):
        keys = idx[h][msk[h] != 0].long() // 16
        cnt = torch.bincount(keys, minlength=nblk)
        steps += int(((cnt + 31) // 32).sum().item())
    del idx, msk
    dkdv = float(B * steps * dkdv_unit)
    return {"dq": dq, "dkdv": dkdv}


def executed_flops(torch, kernel: str, lay, B: int, H: int, L: int, D: int,
                   split: int = 0) -> float:
    """kernel "tile" or "band" over all L rows, or "split": the tile kernel's
    blocks over rows [0, split) and the band kernel's pairs over the rest."""
    if kernel == "tile":
        return B * executed_blocks(torch, lay, L) * 4.0 * 32 * 32 * D
    if kernel == "split":
        band = band_executed_flops(B, H, L, D, W) - band_executed_flops(B, H, split, D, W)
        return B * executed_blocks(torch, lay, split) * 4.0 * 32 * 32 * D + band
    if lay.pattern.layer_idx == 0:
        return window_executed_flops(B, H, L, D, W)  # the band entry point's window kernel
    return band_executed_flops(B, H, L, D, W)


def alg_bytes_of(B: int, H: int, L: int, D: int) -> int:
    """Q, K, V read and O written once in bf16, LSE in float32 (MHA)."""
    return 2 * B * (2 * H * L * D + 2 * H * L * D) + 4 * B * H * L


def bwd_alg_bytes_of(B: int, H: int, Hkv: int, L: int, D: int) -> int:
    """The backward's: Q, O, dO read and dQ written (H heads), K, V read and
    dK, dV written (Hkv heads) once in bf16, LSE read in float32."""
    return 2 * B * L * D * 4 * (H + Hkv) + 4 * B * H * L


def roofline_of(layer: int, kern_ms: float, executed: float, alg_bytes: int, traffic) -> dict:
    if layer == 0:
        # a plain sliding window: ~127 flop/B, below the MFMA ridge -> HBM-bound
        gbs = alg_bytes / (kern_ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic}
    tf = executed / (kern_ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 3), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": traffic}


def profiled_kernel(kernel: str, layer: int) -> str:
    """The kernel whose profiles/ summary covers a prefill: the band entry
    point runs the sliding-window kernel at layer 0."""
    return "window_fwd_kernel" if kernel == "band" and layer == 0 else f"{kernel}_fwd_kernel"


def figure_from_profile(name: str, key: str = "traffic_bytes_per_launch"):
    """A per-launch figure of a kernel (HBM bytes by default) from the
    committed rocprofv3 --pmc summary for this workload (profiles/<name>), or
    None."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith(key + ":"):
                return int(float(line.split(":", 1)[1].strip()))
    return None


def make_inputs(torch, cfg: str, dev, on_device: bool):
    """Seeded q, k, v of a configured workload, bf16 on `dev`: drawn on the
    CPU (the oracle's generator order) or, for the configs object, on the
    GPU (same distribution, faster)."""
    B, H, L, D, scale, outl = CONFIGS[cfg]
    g = torch.Generator(device=dev if on_device else "cpu").manual_seed(0)
    where = dev if on_device else "cpu"
    q = torch.randn(B, H, L, D, generator=g, device=where) * scale
    k = torch.randn(B, H, L, D, generator=g, device=where) * scale
    v = torch.randn(B, H, L, D, generator=g, device=where) * scale
    if outl > 0:
        ch = torch.randperm(D, generator=g, device=where)[:int(math.ceil(outl * D))]
        q[..., ch] *= 20.0
        k[..., ch] *= 20.0
    return q.to(torch.bfloat16).to(dev), k.to(torch.bfloat16).to(dev), v.to(torch.bfloat16).to(dev)


def time_backward(torch, lay, q, k, v, scaling, counted_fwd, steps, warmup) -> dict:
    """The backward (dQ, dK, dV from the forward's O and LSE, with the
    kernels `bwd_kernels` picks) on the same inputs: median of `steps`
    launches (HIP events on the launch stream) after `warmup`; for a
    block-sparse half the tile masks and work lists are built (and cached)
    before timing, as the layout is.  counted_tflops counts 2.5x the
    forward's active-tile flops (QK^T, dP, dV, dK, dQ), the same counted
    convention as the forward's value."""
    from elastic_sparse_attention import bwd_kernels, elastic_attention_bwd, elastic_attention_fwd
    B, H, L, D = q.shape
    o, lse = elastic_attention_fwd(q, k, v, lay, scaling)
    g = torch.Generator(device=q.device).manual_seed(1)
    do = torch.randn(B, L, H, D, generator=g, device=q.device).to(q.dtype)
    kinds = bwd_kernels(lay, L, B, D)
    t0 = time.perf_counter()
    if kinds[1] == "tile":
        lay.tile_masks(L)
        lay.bwd_plan(L, B, k.shape[1])
    if kinds[0] == "tile":
        lay.schedule(L, B)
    torch.cuda.synchronize()
    setup_ms = (time.perf_counter() - t0) * 1e3
    ms = event_ms(torch, lambda: elastic_attention_bwd(q, k, v, o, lse, do, lay, scaling),
                  steps, warmup)
    out = {"ms": round(ms, 4),
           "counted_tflops": round(2.5 * counted_fwd / (ms * 1e-3) / 1e12, 3),
           "flops_convention": "2.5 x forward active-tile flops (counted, not executed)",
           "kernels": {"dq": kinds[0], "dkdv": kinds[1]},
           "mask_and_plan_setup_ms": round(setup_ms, 2)}
    if kinds == ("band", "band"):
        ex = band_bwd_executed_flops(torch, lay, B, H, k.shape[1], L, D, W)
        tf = (ex["dq"] + ex["dkdv"]) / (ms * 1e-3) / 1e12
        out["executed_mfma_flops"] = {"dq": ex["dq"], "dkdv": ex["dkdv"]}
        if lay.pattern.layer_idx == 0:
            # a sliding window: HBM-bound (about 85 executed flop per
            # algorithmic byte); the backward's algorithmic bytes over its time
            alg = bwd_alg_bytes_of(B, H, k.shape[1], L, D)
            gbs = alg / (ms * 1e-3) / 1e9
            out["algorithmic_bytes"] = alg
            out["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                               "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4)}
        else:
            # executed bf16 MFMA work of both kernels over the whole backward's
            # time (per-kernel rates: the committed trace and counter summary)
            out["roofline"] = {"bound": "mfma", "achieved": round(tf, 3),
                               "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                               "frac": round(tf / PEAK_BF16_TFLOPS, 4)}
        prof = f"band_bwd_kernels_bf16_B{B}_H{H}_L{L}_D{D}_layer{lay.pattern.layer_idx}.md"
        l2 = figure_from_profile(prof, "l2_to_cu_bytes_per_launch")
        hbm = figure_from_profile(prof)
        if l2 is not None:
            out["l2_to_cu_bytes"] = l2
        if hbm is not None:
            out["traffic"] = hbm
            if out["roofline"]["bound"] == "hbm":
                out["roofline"]["traffic"] = hbm
    return out


def one_config(torch, cfg: str, layer: int, dev, steps: int, warmup: int, with_bwd: bool) -> dict:
    """Forward (and backward) kernel time of one configured workload and
    layer, through the module's kernel choice."""
    from elastic_sparse_attention import ElasticSparseAttention, elastic_attention_fwd, prefill_split
    B, H, L, D, _, _ = CONFIGS[cfg]
    q, k, v = make_inputs(torch, cfg, dev, on_device=True)
    m = ElasticSparseAttention(layer_idx=layer, num_hidden_layers=NL, num_attention_heads=H,
                               head_dim=D, attention_length=W, max_seq_len=L)
    lay = m.layout(dev)
    split = prefill_split(lay, L, B, D)
    kernel = "band" if split == 0 else ("tile" if split == L else "split")
    if kernel != "band":
        lay.stages(64, 128).schedule(split, B)
        lay.stages(64, 128).stage_masks()
    counted = lay.tiles_for(L) * B * 4.0 * 128 * 128 * D
    with torch.no_grad():
        ms = event_ms(torch, lambda: elastic_attention_fwd(q, k, v, lay, m.scaling,
                                                           return_lse=False),
                      steps, warmup)
    executed = executed_flops(torch, kernel, lay, B, H, L, D, split)
    prof = f"{profiled_kernel(kernel, layer)}_bf16_B{B}_H{H}_L{L}_D{D}_layer{layer}_pmc.md"
    out = {"workload": f"bf16 B={B} H={H} L={L} D={D}, w={W}, layer {layer} of {NL}",
           "kernel": kernel, "fwd_ms": round(ms, 4),
           "counted_tflops": round(counted / (ms * 1e-3) / 1e12, 3),
           "executed_flop_fraction": round(executed / counted, 4),
           "roofline": roofline_of(layer, ms, executed, alg_bytes_of(B, H, L, D),
                                   figure_from_profile(prof))}
    if kernel == "split":
        out["split_row"] = split  # tile kernel on rows [0, split), band kernel on the rest
    if with_bwd:
        try:
            bwd = time_backward(torch, lay, q, k, v, m.scaling, counted, steps, warmup)
            out["bwd_ms"] = bwd["ms"]
            out["bwd_kernels"] = bwd["kernels"]
        except Exception as exc:  # noqa: BLE001
            out["bwd_error"] = f"{type(exc).__name__}: {exc}"
    del q, k, v, m, lay
    torch.cuda.empty_cache()
    return out


DECODE = (128, 32, 8, 32768, 128)  # batch, query heads, kv heads, cache length, head dim


def time_decode(torch, layer: int, steps: int, warmup: int) -> dict:
    """One decode step of a serving batch: B sequences, one new query row
    each at position L - 1 of a cache of L keys (GQA 32 / 8, bf16), through
    the module's forward(q, k_cache, v_cache, cache_position=...) (the
    per-row gather kernel), `steps` calls back to back between two HIP
    events on the launch stream, so the per-call host cost is in the time.
    Bytes: the w K rows and w V rows each (batch, head) gathers, plus Q and
    O."""
    from elastic_sparse_attention import ElasticSparseAttention
    B, H, Hkv, L, D = DECODE
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(3)
    k = torch.randn(B, Hkv, L, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, L, D, device=dev, generator=g).to(torch.bfloat16)
    q = (torch.randn(B, H, 1, D, device=dev, generator=g) * D ** -0.25).to(torch.bfloat16)
    m = ElasticSparseAttention(layer_idx=layer, num_hidden_layers=NL, num_attention_heads=H,
                               head_dim=D, attention_length=W, max_seq_len=L,
                               num_key_value_heads=Hkv)
    pos = torch.tensor([L - 1], dtype=torch.int64, device=dev)

    def call():
        m(q, k, v, cache_position=pos)

    with torch.no_grad():
        for _ in range(warmup):
            call()
        stream = torch.cuda.current_stream(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(steps):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    nbytes = B * H * W * D * 2 * 2 + 2 * B * H * D * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"workload": (f"decode step through the module (cache_position), bf16, B={B} "
                         f"sequences x 1 row, H={H} Hkv={Hkv}, cache L={L}, D={D}, w={W}, "
                         f"layer {layer} of {NL}"),
            "us_per_step": round(us, 2), "rows_per_s": round(B / (us * 1e-6)),
            "gathered_bytes": nbytes,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4)}}


CHUNK = (28672, 4096)  # a chunked prefill of the headline shape: rows p0 .. p0 + n - 1


def time_chunk(torch, cfg: str, layer: int, steps: int, warmup: int) -> dict:
    """A chunked prefill through the module: the last CHUNK rows of a
    configured sequence as query rows with cache_position = arange(p0, p0 +
    n) on the device, against the full key/value cache (the band kernel at
    the given positions).  Beside it, the same rows' share of a full prefill
    (the band kernel does the same work for every 16-row group, so the share
    is the full forward's time times n / L)."""
    from elastic_sparse_attention import ElasticSparseAttention, elastic_attention_band
    B, H, L, D, _, _ = CONFIGS[cfg]
    p0, n = CHUNK
    dev = torch.device("cuda", 0)
    q, k, v = make_inputs(torch, cfg, dev, on_device=True)
    m = ElasticSparseAttention(layer_idx=layer, num_hidden_layers=NL, num_attention_heads=H,
                               head_dim=D, attention_length=W, max_seq_len=L)
    qc = q[:, :, p0:p0 + n].contiguous()
    pos = torch.arange(p0, p0 + n, dtype=torch.int64, device=dev)
    with torch.no_grad():
        chunk_ms = event_ms(torch, lambda: m(qc, k, v, cache_position=pos), steps, warmup)
        full_ms = event_ms(torch, lambda: elastic_attention_band(q, k, v, m.pattern, m.scaling,
                                                                 return_lse=False),
                           steps, warmup)
    share = full_ms * n / L
    del q, k, v, qc
    torch.cuda.empty_cache()
    return {"workload": (f"chunked prefill through the module (cache_position = arange({p0}, "
                         f"{p0 + n})), bf16 B={B} H={H} kv L={L} D={D}, w={W}, layer {layer} "
                         f"of {NL}"),
            "chunk_ms": round(chunk_ms, 4), "full_prefill_ms": round(full_ms, 4),
            "prefill_rows_share_ms": round(share, 4),
            "ratio_to_prefill_share": round(chunk_ms / share, 3)}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--config", default="32k", choices=sorted(CONFIGS))
    ap.add_argument("--layer", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel", default="auto", choices=["auto", "band", "tile"],
                    help="prefill kernel the module runs (default: the faster for the shape)")
    ap.add_argument("--no-backward", dest="backward", action="store_false",
                    help="skip timing the backward (reported beside the forward by default)")
    ap.add_argument("--no-decode", dest="decode", action="store_false",
                    help="skip timing one decode step of a serving batch (reported by default)")
    ap.add_argument("--no-configs", dest="configs", action="store_false",
                    help="skip the per-configuration forward/backward table")
    ap.add_argument("--no-chunk", dest="chunk", action="store_false",
                    help="skip timing a chunked prefill (cache_position rows) of the headline")
    ap.add_argument("--config-steps", type=int, default=20)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain device copy of known size (HBM counter scale)")
    ap.add_argument("--peaks", action="store_true",
                    help="run only the rate probes (bf16 MFMA, HBM read, copy, L2 -> LDS)")
    ap.add_argument("--lds-probe", action="store_true",
                    help="run only the band kernels' LDS operand-read probes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU: every box here has one, "
                          "and the forward is a single-device kernel (sharding over heads or "
                          "sequence is design-only)", "n_gpus": args.gpus}), flush=True)
        sys.exit(2)

    import torch
    if args.copy_calibration:
        copy_calibration(torch)
        return
    if args.peaks:
        peaks(torch)
        return
    if args.lds_probe:
        print(json.dumps({"lds_read": lds_probe(torch)}), flush=True)
        return
    from elastic_sparse_attention import ElasticSparseAttention, prefill_split

    B, H, L, D, _, _ = CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    q, k, v = make_inputs(torch, args.config, dev, on_device=False)

    m = ElasticSparseAttention(layer_idx=args.layer, num_hidden_layers=NL,
                               num_attention_heads=H, head_dim=D, attention_length=W,
                               max_seq_len=L)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    lay = m.layout(dev)           # 128 x 128 tiles: the declared (counted) tile
    # the module's choice: one kernel, or the tile kernel on rows [0, split)
    # and the band kernel on the rest
    split = prefill_split(lay, L, B, D) if args.kernel == "auto" else \
        (0 if args.kernel == "band" else L)
    kernel = "band" if split == 0 else ("tile" if split == L else "split")
    if kernel != "band":
        st = lay.stages(64, 128)      # 128 x 64 blocks: the tile kernel's staging unit
        st.schedule(split, B)
        if args.layer > 0:
            st.stage_masks()          # per-stage row masks, once per pattern
    m.prefill_kernel = "auto" if kernel == "split" else kernel
    torch.cuda.synchronize()
    layout_ms = (time.perf_counter() - t0) * 1e3

    tiles = lay.tiles_for(L) * B
    counted = tiles * 4.0 * 128 * 128 * D
    nnz = H * sum(min(i + 1, W) for i in range(L)) * B
    useful = 4.0 * D * nnz
    alg_bytes = alg_bytes_of(B, H, L, D)

    with torch.no_grad():
        t0 = time.perf_counter()
        for _ in range(args.warmup):
            m(q, k, v)
        torch.cuda.synchronize()
        while (time.perf_counter() - t0) * 1e3 < WARM_MS:  # clocks up before timing
            m(q, k, v)
            torch.cuda.synchronize()
        # timed region: K forwards, each bracketed by HIP events on the stream
        # the module launches on (torch's current stream), wall clock around all K
        stream = torch.cuda.current_stream(dev)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.steps)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s_ev, e_ev in evs:
            s_ev.record(stream)
            m(q, k, v)
            e_ev.record(stream)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / args.steps
    kern_ms = statistics.mean(s.elapsed_time(e) for s, e in evs)

    value = counted / wall / 1e12
    executed = executed_flops(torch, kernel, lay, B, H, L, D, split)
    prof = f"{profiled_kernel(kernel, args.layer)}_bf16_B{B}_H{H}_L{L}_D{D}_layer{args.layer}_pmc.md"
    traffic = figure_from_profile(prof)
    l2_bytes = figure_from_profile(prof, "l2_to_cu_bytes_per_launch")
    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs of the configured shape)",
        "config": {"workload": (f"elastic block-sparse attention forward, bf16, B={B} H={H} "
                                f"L={L} D={D}, w={W}, layer {args.layer} of {NL}, "
                                f"128x128 tiles"),
                   "batch": B, "heads": H, "seq_len": L, "head_dim": D,
                   "attention_length": W, "layer_idx": args.layer, "num_hidden_layers": NL,
                   "block": [128, 128], "active_tiles": tiles, "kernel": kernel,
                   **({"split_row": split} if kernel == "split" else {})},
        "counted_pct_of_bf16_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "kernel_ms": round(kern_ms, 4),
        "executed_flop_fraction": round(executed / counted, 4),
        "executed_mfma_tflops": round(executed / (kern_ms * 1e-3) / 1e12, 3),
        "useful_tflops": round(useful / wall / 1e12, 4),
        "hbm_gbs_algorithmic": round(alg_bytes / (kern_ms * 1e-3) / 1e9, 1),
        "layout_build_ms": round(layout_ms, 2),
        "roofline": roofline_of(args.layer, kern_ms, executed, alg_bytes, traffic),
        "cpu_baseline": None,
    }
    if l2_bytes is not None:
        tbs = l2_bytes / (kern_ms * 1e-3) / 1e12
        try:
            import esa_native as en
            rates = l2_lds_rates(torch, en.load_probe(), 5, pers=(8,))
            ceil = rates["gather"]["tbs"]
            out["l2_to_cu"] = {"achieved": round(tbs, 2), "ceiling": ceil, "unit": "TB/s",
                               "frac": round(tbs / ceil, 4), "bytes": l2_bytes,
                               "ceiling_probe": "256-byte rows at random positions of a 1 MiB "
                                                "L2-resident region into LDS, 8 workgroups "
                                                "per CU, measured in this run",
                               "stream_tbs": rates["stream"]["tbs"]}
        except Exception as exc:  # noqa: BLE001
            out["l2_to_cu"] = {"achieved": round(tbs, 2), "bytes": l2_bytes,
                               "error": f"{type(exc).__name__}: {exc}"}
    # the side measurements never cost the headline line: a failure is reported
    if args.backward:
        try:
            out["backward"] = time_backward(torch, lay, q, k, v, m.scaling, counted, args.steps,
                                            args.warmup)
        except Exception as exc:  # noqa: BLE001
            out["backward"] = {"error": f"{type(exc).__name__}: {exc}"}
    del q, k, v
    torch.cuda.empty_cache()
    if args.configs:
        rows = {}
        for cfg, layers in CONFIG_LAYERS.items():
            for layer in layers:
                key = f"{cfg}/layer{layer}"
                try:
                    rows[key] = one_config(torch, cfg, layer, dev, args.config_steps, 5,
                                           args.backward)
                except Exception as exc:  # noqa: BLE001
                    rows[key] = {"error": f"{type(exc).__name__}: {exc}"}
                print(f"# configs {key}: {rows[key].get('fwd_ms')} ms", file=sys.stderr,
                      flush=True)
        out["configs"] = rows
    if args.chunk:
        try:
            out["chunked_prefill"] = time_chunk(torch, "32k", args.layer, args.steps, args.warmup)
        except Exception as exc:  # noqa: BLE001
            out["chunked_prefill"] = {"error": f"{type(exc).__name__}: {exc}"}
    if args.decode:
        try:
            out["decode"] = time_decode(torch, args.layer, max(args.steps, 50), args.warmup)
        except Exception as exc:  # noqa: BLE001
            out["decode"] = {"error": f"{type(exc).__name__}: {exc}"}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.config, args.layer, counted)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
