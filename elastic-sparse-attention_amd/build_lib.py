"""Builds libesa.so (the HIP kernels and the C ABI) and libesa_probe.so (the
rate probes bench.py --peaks runs) for gfx950 in place.

    python elastic-sparse-attention_amd/build_lib.py [-v] [--sanitize]

--sanitize builds libesa_san.so instead: the same sources with the host code
under AddressSanitizer and UndefinedBehaviorSanitizer (device code is left
alone), for running the host-side tests against (tests/test_sanitizers.py);
esa_native loads it when ESA_LIB names it.

hipcc cross-compiles without a GPU.  Each source is compiled to an object
(in parallel) under _build/ next to this file, then the objects are linked
into libesa.so and libesa_probe.so, which land next to this file, where
esa_native.py loads them from.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
SOURCES = ["esa_capi.hip", "esa_layout.hip", "esa_fwd_tile.hip", "esa_fwd_band.hip",
           "esa_bwd_band.hip", "esa_fwd_gather.hip", "esa_bwd_gather.hip", "esa_bwd.hip",
           "esa_reach.hip", "esa_bwd_fix.hip", "esa_fwd_window.hip"]
PROBE_SOURCES = ["esa_probe.hip"]
LIB = os.path.join(HERE, "libesa.so")
PROBE_LIB = os.path.join(HERE, "libesa_probe.so")
SAN_LIB = os.path.join(HERE, "libesa_san.so")
SAN_BUILD = os.path.join(HERE, "_build_san")
# host-only sanitizers: each -fsanitize= applies to the host pass alone
SAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host",
             "-fno-omit-frame-pointer", "-g"]
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
         # packed fp32 VALU forms are kept out of every kernel
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-result"]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libesa.so")


def _messages(res: subprocess.CompletedProcess) -> list:
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    return [ln for ln in (res.stdout + res.stderr).splitlines()
            if "packed-fp32-ops" not in ln and ln.strip()]


def _compile(src: str, verbose: bool, san: bool = False) -> str:
    obj = os.path.join(SAN_BUILD if san else BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *FLAGS, *(SAN_FLAGS if san else []), "-I",
           os.path.join(HERE, "..", "include"), "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    msgs = _messages(res)
    if res.returncode != 0:
        raise RuntimeError(f"compiling {src} failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)
    return obj


def _link(objs: list, lib: str, verbose: bool, san: bool = False) -> None:
    tmp = lib + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC",
           *(["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
              "-shared-libsan"] if san else []), *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking {os.path.basename(lib)} failed:\n" +
                           "\n".join(_messages(res)))
    os.replace(tmp, lib)


def build(verbose: bool = False) -> str:
    """Compiles every source, links libesa.so and libesa_probe.so; returns
    libesa.so's path."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = SOURCES + PROBE_SOURCES
    workers = min(len(srcs), max(1, min(os.cpu_count() or 1, 8)))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    _link(objs[:len(SOURCES)], LIB, verbose)
    _link(objs[len(SOURCES):], PROBE_LIB, verbose)
    return LIB


def build_sanitized(verbose: bool = False) -> str:
    """Compiles every library source with host-side ASan/UBSan and links
    libesa_san.so; returns its path."""
    os.makedirs(SAN_BUILD, exist_ok=True)
    workers = min(len(SOURCES), max(1, min(os.cpu_count() or 1, 8)))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, san=True), SOURCES))
    _link(objs, SAN_LIB, verbose, san=True)
    return SAN_LIB


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        print(build_sanitized(verbose="-v" in sys.argv))
    else:
        print(build(verbose="-v" in sys.argv))
