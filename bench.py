"""Benchmark: elastic block-sparse attention forward on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config 32k|8k|batched|128k]
                    [--layer N] [--no-cpu] [--no-backward] [--no-decode]

A step is one ElasticSparseAttention.forward over one batch of synthetic
input already resident in HBM (the module's drop-in HIP path: one kernel
launch, the band-gathered kernel or the block-sparse tile kernel, whichever
is faster for the shape; config.kernel names it).  The block layout is built
before the timed region, as the reference builds its index cache at
construction; its build time is reported separately.

Prints ONE JSON line.  value = counted active-tile flops / wall time per
step, where counted flops = active 128x128 tiles x 4 * 128 * 128 * D (the
metric's unit of work, whatever the kernel executes).  roofline.achieved
uses the same flops over the kernel's own average duration (HIP events on the
launch stream).  The kernels issue far fewer MFMA flops than that: the tile
kernel only the 32 x 32 blocks of an active tile that hold a valid key for
one of a wave's rows, the band kernel 16 keys x 16 rows per entry of the
rows' index lists; executed_flop_fraction and executed_mfma_tflops report
that work.  What bounds both at dilated layers is the K/V they gather from
L2: l2_to_cu gives those bytes (from the committed rocprofv3 summary) over
the kernel's time, against the L2 -> CU rate a copy kernel reaches.  cpu_baseline times the reference's
PyTorch fallback (_naive_forward, restated in oracle/) on the host cores on a
bounded sample of query rows of the same workload, extrapolated linearly
(every row costs the same w-key gather there).  Reported beside the forward
(skipped with the flags above): "backward", the backward of the same
forward (dQ, dK, dV from its O and LSE) with the kernels bwd_kernels picks,
and "decode", one decode step of 128 sequences (GQA 32 / 8, 32K-key cache)
through the per-row gather, against HBM bandwidth.
"""
from __future__ import annotations

import argparse
import json
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
W, NL = 64, 8
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
METRIC = "active-block TFLOP/s + % of bf16 MFMA peak, elastic attn fwd, 1 GPU, L=32K"


def cpu_baseline(cfg_name: str, layer: int, counted_flops: float, rows_per_run: int = 2048,
                 runs: int = 3) -> dict:
    """The reference's PyTorch fallback on the host, on every (L / rows)-th
    query row, all heads, full K/V; median of `runs` after one warm-up."""
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from esa_oracle import elastic_indices, naive_forward, seeded_inputs

    B, H, L, D, scale, outl = CONFIGS[cfg_name]
    cores = torch.get_num_threads()  # OMP_NUM_THREADS, else the host's cores
    q, k, v = seeded_inputs(B, H, H, L, D, torch.bfloat16, seed=0, scale=scale,
                            outlier_frac=outl)
    t0 = time.perf_counter()
    idx, msk = elastic_indices(L, layer, NL, H, W)
    layout_s = time.perf_counter() - t0
    stride = max(1, L // rows_per_run)
    pos = torch.arange(0, L, stride)[:rows_per_run]
    qs = q[:, :, pos].contiguous()
    naive_forward(qs[:, :, :256], k, v, idx, msk, D ** -0.5, 1, L, cache_position=pos[:256],
                  chunk_rows=256)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        naive_forward(qs, k, v, idx, msk, D ** -0.5, 1, L, cache_position=pos, chunk_rows=256)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    full_s = t * L / len(pos)
    return {"value": counted_flops / full_s / 1e12, "unit": "TFLOP/s", "cores": cores,
            "kind": "port",
            "sample": (f"reference PyTorch fallback (_naive_forward restated, bf16) on "
                       f"{len(pos)} of {L} query rows (every {stride}th), all {H} heads, "
                       f"B={B}; median of {runs} runs = {t:.2f} s, extrapolated to "
                       f"{full_s:.1f} s per forward"),
            "seconds_per_forward": full_s, "layout_build_s": layout_s}


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


def time_backward(torch, m, q, k, v, lay, counted_fwd, steps, warmup) -> dict:
    """The backward (dQ, dK, dV from the forward's O and LSE, with the
    kernels `bwd_kernels` picks) on the same inputs: mean of `steps` launches
    (HIP events on the launch stream) after `warmup`; for a block-sparse
    half the tile masks and work lists are built (and cached) before timing,
    as the layout is.  TFLOP/s counts 2.5x the forward's active-tile flops
    (QK^T, dP, dV, dK, dQ)."""
    from elastic_sparse_attention import bwd_kernels, elastic_attention_bwd, elastic_attention_fwd
    B, H, L, D = q.shape
    o, lse = elastic_attention_fwd(q, k, v, lay, m.scaling)
    g = torch.Generator(device="cpu").manual_seed(1)
    do = torch.randn(B, L, H, D, generator=g).to(q.dtype).to(q.device)
    kinds = bwd_kernels(lay, L, B, D)
    t0 = time.perf_counter()
    if kinds[1] == "tile":
        lay.tile_masks(L)
        lay.bwd_plan(L, B, k.shape[1])
    if kinds[0] == "tile":
        lay.schedule(L, B)
    torch.cuda.synchronize()
    setup_ms = (time.perf_counter() - t0) * 1e3
    for _ in range(warmup):
        elastic_attention_bwd(q, k, v, o, lse, do, lay, m.scaling)
    stream = torch.cuda.current_stream(q.device)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    torch.cuda.synchronize()
    for s_ev, e_ev in evs:
        s_ev.record(stream)
        elastic_attention_bwd(q, k, v, o, lse, do, lay, m.scaling)
        e_ev.record(stream)
    torch.cuda.synchronize()
    ms = statistics.mean(a.elapsed_time(b) for a, b in evs)
    return {"ms": round(ms, 4), "tflops": round(2.5 * counted_fwd / (ms * 1e-3) / 1e12, 3),
            "flops_convention": "2.5 x forward active-tile flops",
            "kernels": {"dq": kinds[0], "dkdv": kinds[1]},
            "mask_and_plan_setup_ms": round(setup_ms, 2)}


DECODE = (128, 32, 8, 32768, 128)  # batch, query heads, kv heads, cache length, head dim


def time_decode(torch, layer: int, steps: int, warmup: int) -> dict:
    """One decode step of a serving batch: B sequences, one new query row
    each at position L - 1 of a cache of L keys (GQA 32 / 8, bf16), through
    esa_elastic_fwd_rows (the path the module's cache_position branch takes).
    The C entry point is called directly with prebuilt arguments, `steps`
    times back to back between two HIP events on the launch stream, so the
    host's per-call cost (a few us) stays below the kernel's.  Bytes: the
    w K rows and w V rows each (batch, head) gathers, plus Q and O."""
    import ctypes
    from elastic_sparse_attention import _fwd_args, _stream, make_pattern
    from esa_native import check, load
    B, H, Hkv, L, D = DECODE
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(3)
    k = torch.randn(B, Hkv, L, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, L, D, device=dev, generator=g).to(torch.bfloat16)
    q = (torch.randn(B, H, 1, D, device=dev, generator=g) * D ** -0.25).to(torch.bfloat16)
    o = torch.empty(B, 1, H, D, dtype=torch.bfloat16, device=dev)
    pat = make_pattern(L, W, layer, NL, H)
    pos = torch.tensor([L - 1], dtype=torch.int64, device=dev)
    a = _fwd_args(q, k, v, o, (o.stride(0), o.stride(2), o.stride(1)), None, D ** -0.5)
    lib = load()
    st = _stream(dev)
    pp = ctypes.c_void_p(pos.data_ptr())

    def call():
        check(lib.esa_elastic_fwd_rows(ctypes.byref(a), ctypes.byref(pat), pp, st),
              "esa_elastic_fwd_rows")

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
    return {"workload": (f"decode step, bf16, B={B} sequences x 1 row, H={H} Hkv={Hkv}, "
                         f"cache L={L}, D={D}, w={W}, layer {layer} of {NL}"),
            "us_per_step": round(us, 2), "rows_per_s": round(B / (us * 1e-6)),
            "gathered_bytes": nbytes,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4)}}


def executed_blocks(torch, lay, L: int) -> int:
    """Number of (active tile, 32-row block, 32-key block) triples in which
    some row has a valid key, per batch element: the blocks the forward
    issues MFMAs for.  From the layout's key-major tile masks (32 row bits per
    key), built here after the timed region."""
    masks = lay.tile_masks(L)
    n = lay.num_tiles  # every tile of the layout; rows at or past L carry no bits
    return int(masks[:n * 512].view(n, 4, 4, 32).ne(0).any(-1).sum().item())


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


def figure_from_profile(name: str, key: str = "traffic_bytes_per_launch"):
    """A per-launch figure of the forward kernel (HBM bytes by default) from
    the committed rocprofv3 --pmc summary for this workload
    (profiles/<name>), or None."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith(key + ":"):
                return int(float(line.split(":", 1)[1].strip()))
    return None


# L2 -> CU streaming rate of MI355X measured with a copy kernel reading 4 KB
# row blocks from an L2-resident buffer (buffer_load ... lds or into
# registers, 4-10 waves per CU): the ceiling of the gather-bound forwards
L2_TO_CU_TBS = 36.0


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="32k", choices=sorted(CONFIGS))
    ap.add_argument("--layer", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel", default="auto", choices=["auto", "band", "tile"],
                    help="prefill kernel the module runs (default: the faster for the shape)")
    ap.add_argument("--no-backward", dest="backward", action="store_false",
                    help="skip timing the backward (reported beside the forward by default)")
    ap.add_argument("--backward", action="store_true", default=True,
                    help=argparse.SUPPRESS)
    ap.add_argument("--no-decode", dest="decode", action="store_false",
                    help="skip timing one decode step of a serving batch (reported by default)")
    ap.add_argument("--decode", action="store_true", default=True, help=argparse.SUPPRESS)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain device copy of known size (HBM counter scale)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU; the forward is a "
                          "single-device kernel (multi-GPU sharding is design-only)",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    if args.copy_calibration:
        copy_calibration(torch)
        return
    from elastic_sparse_attention import ElasticSparseAttention, prefill_kernel

    B, H, L, D, scale, outl = CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    g = torch.Generator(device="cpu").manual_seed(0)
    q = (torch.randn(B, H, L, D, generator=g) * scale)
    k = (torch.randn(B, H, L, D, generator=g) * scale)
    v = (torch.randn(B, H, L, D, generator=g) * scale)
    if outl > 0:
        import math
        ch = torch.randperm(D, generator=g)[:int(math.ceil(outl * D))]
        q[..., ch] *= 20.0
        k[..., ch] *= 20.0
    q = q.to(torch.bfloat16).to(dev)
    k = k.to(torch.bfloat16).to(dev)
    v = v.to(torch.bfloat16).to(dev)

    m = ElasticSparseAttention(layer_idx=args.layer, num_hidden_layers=NL,
                               num_attention_heads=H, head_dim=D, attention_length=W,
                               max_seq_len=L)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    lay = m.layout(dev)           # 128 x 128 tiles: the declared (counted) tile
    lay.stages().schedule(L, B)   # 64 x 32 blocks: the tile kernel's staging unit
    kernel = prefill_kernel(lay, L, B, D) if args.kernel == "auto" else args.kernel
    m.prefill_kernel = kernel
    torch.cuda.synchronize()
    layout_ms = (time.perf_counter() - t0) * 1e3

    tiles = lay.tiles_for(L) * B
    counted = tiles * 4.0 * 128 * 128 * D
    nnz = H * sum(min(i + 1, W) for i in range(L)) * B
    useful = 4.0 * D * nnz
    alg_bytes = 2 * B * (2 * H * L * D + 2 * H * L * D) + 4 * B * H * L

    for _ in range(args.warmup):
        m(q, k, v)
    torch.cuda.synchronize()
    # timed region: K forwards, each bracketed by HIP events on the stream the
    # module launches on (torch's current stream), wall clock around all K
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

    achieved = counted / (kern_ms * 1e-3) / 1e12
    value = counted / wall / 1e12
    if kernel == "tile":
        # MFMA work actually issued: inside each active tile a wave skips the
        # 32 x 32 (rows x keys) blocks where none of its rows has a valid key
        executed = B * executed_blocks(torch, lay, L) * 4.0 * 32 * 32 * D
    else:
        executed = band_executed_flops(B, H, L, D, W)
    prof = f"{kernel}_fwd_kernel_bf16_B{B}_H{H}_L{L}_D{D}_layer{args.layer}_pmc.md"
    traffic = figure_from_profile(prof)
    l2_bytes = figure_from_profile(prof, "l2_to_cu_bytes_per_launch")
    if args.layer == 0:
        # a plain sliding window: ~127 flop/B, below the MFMA ridge -> HBM-bound
        gbs = alg_bytes / (kern_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic}
    else:
        roofline = {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_BF16_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                    "traffic": traffic}
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
                   "staged_blocks_64x32": lay.stages().num_tiles * B},
        "pct_of_bf16_mfma_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "kernel_ms": round(kern_ms, 4),
        "executed_flop_fraction": round(executed / counted, 4),
        "executed_mfma_tflops": round(executed / (kern_ms * 1e-3) / 1e12, 3),
        "useful_tflops": round(useful / wall / 1e12, 4),
        "hbm_gbs_algorithmic": round(alg_bytes / (kern_ms * 1e-3) / 1e9, 1),
        "layout_build_ms": round(layout_ms, 2),
        "roofline": roofline,
        "cpu_baseline": None,
    }
    if l2_bytes is not None:
        # what bounds the kernel at dilated layers: bytes it gathers from L2
        # (profiled) over its measured time, against the probe's ceiling
        tbs = l2_bytes / (kern_ms * 1e-3) / 1e12
        out["l2_to_cu"] = {"achieved": round(tbs, 2), "ceiling": L2_TO_CU_TBS, "unit": "TB/s",
                           "frac": round(tbs / L2_TO_CU_TBS, 4), "bytes": l2_bytes}
    # the side measurements never cost the headline line: a failure is reported
    if args.backward:
        try:
            out["backward"] = time_backward(torch, m, q, k, v, lay, counted, args.steps,
                                            args.warmup)
        except Exception as exc:  # noqa: BLE001
            out["backward"] = {"error": f"{type(exc).__name__}: {exc}"}
    if args.decode:
        del q, k, v
        torch.cuda.empty_cache()
        try:
            out["decode"] = time_decode(torch, args.layer, max(args.steps, 50), args.warmup)
        except Exception as exc:  # noqa: BLE001
            out["decode"] = {"error": f"{type(exc).__name__}: {exc}"}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.config, args.layer, counted)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
