"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only).

elastic-sparse-attention_amd/build_lib.py --sanitize builds libesa_san.so:
the same sources with the host pass instrumented (device code untouched).
This runs tests/test_capi.py (the host-only entry points: esa_layout_sizes,
esa_plan_schedule, esa_plan_bwd, esa_stage_masks_size, the workspace sizes,
and every entry point's argument checks) against it in a child process that
preloads the sanitizer runtime; any report aborts the child.
"""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_LIB = os.path.join(ROOT, "elastic-sparse-attention_amd", "libesa_san.so")


def asan_runtime():
    for cand in (shutil.which("clang++"), "/opt/rocm/llvm/bin/clang++"):
        if cand and os.path.exists(cand):
            out = subprocess.run([cand, "--print-file-name=libclang_rt.asan-x86_64.so"],
                                 capture_output=True, text=True).stdout.strip()
            if out and os.path.exists(out):
                return out
    return None


@pytest.mark.skipif(not os.path.exists(SAN_LIB),
                    reason="libesa_san.so not built (build_lib.py --sanitize)")
def test_capi_host_code_under_asan_ubsan():
    rt = asan_runtime()
    if rt is None:
        pytest.skip("the clang AddressSanitizer runtime is not installed")
    env = dict(os.environ, ESA_LIB=SAN_LIB, LD_PRELOAD=rt,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    res = subprocess.run([sys.executable, "-m", "pytest", os.path.join(ROOT, "tests", "test_capi.py"),
                          "-m", "not gpu", "-q", "-p", "no:cacheprovider"],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    tail = (res.stdout + res.stderr)[-3000:]
    assert res.returncode == 0, tail
    assert "AddressSanitizer" not in tail and "runtime error" not in tail, tail
    assert " passed" in tail, tail
