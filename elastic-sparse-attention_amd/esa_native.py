"""ctypes binding of libesa.so (include/esa.h).

Loads the in-tree library built by build_lib.py.  There is no fallback: if
the library is missing the import of the module that needs it fails with an
error naming the build command.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
# ESA_LIB may name another build of the library (the sanitizer build the
# host-side tests run against); by default the in-tree libesa.so
LIB_PATH = os.environ.get("ESA_LIB") or os.path.join(HERE, "libesa.so")
PROBE_LIB_PATH = os.path.join(HERE, "libesa_probe.so")

ESA_OK = 0
ESA_ERR_NULL = 1
ESA_ERR_SHAPE = 2
ESA_ERR_DTYPE = 3
ESA_ERR_ALIGN = 4
ESA_ERR_UNSUPPORTED = 5
ESA_ERR_CAPACITY = 6
ESA_ERR_HIP = 7

ESA_F32 = 0
ESA_BF16 = 1
ESA_F16 = 2

EXPORTED = (
    "esa_status_string", "esa_version", "esa_layout_sizes", "esa_build_indices",
    "esa_build_layout", "esa_plan_schedule", "esa_elastic_fwd", "esa_stage_masks_size",
    "esa_build_stage_masks", "esa_elastic_fwd_band",
    "esa_elastic_fwd_rows",
    "esa_sparse_fwd", "esa_plan_bwd", "esa_build_tile_masks", "esa_bwd_workspace_size",
    "esa_elastic_bwd", "esa_elastic_bwd_noalloc", "esa_bwd_noalloc_max_workspace",
    "esa_init_device", "esa_build_dense_mask",
    "esa_elastic_fwd_naive", "esa_gather_bwd_workspace_size", "esa_sparse_bwd",
    "esa_elastic_bwd_rows", "esa_reachability",
)


class EsaPattern(ctypes.Structure):
    _fields_ = [
        ("seq_len", ctypes.c_int32),
        ("attention_length", ctypes.c_int32),
        ("layer_idx", ctypes.c_int32),
        ("num_hidden_layers", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("block_m", ctypes.c_int32),
        ("block_n", ctypes.c_int32),
    ]


class EsaFwdArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("q_len", ctypes.c_int32),
        ("kv_len", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("q_stride_b", ctypes.c_int64), ("q_stride_h", ctypes.c_int64), ("q_stride_s", ctypes.c_int64),
        ("k", ctypes.c_void_p),
        ("k_stride_b", ctypes.c_int64), ("k_stride_h", ctypes.c_int64), ("k_stride_s", ctypes.c_int64),
        ("v", ctypes.c_void_p),
        ("v_stride_b", ctypes.c_int64), ("v_stride_h", ctypes.c_int64), ("v_stride_s", ctypes.c_int64),
        ("o", ctypes.c_void_p),
        ("o_stride_b", ctypes.c_int64), ("o_stride_h", ctypes.c_int64), ("o_stride_s", ctypes.c_int64),
        ("lse", ctypes.c_void_p),
        ("lse_stride_b", ctypes.c_int64), ("lse_stride_h", ctypes.c_int64),
        ("sm_scale", ctypes.c_float),
    ]


class EsaBwdArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("q_len", ctypes.c_int32),
        ("kv_len", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
    ] + [f for name in ("q", "k", "v", "o", "dout", "dq", "dk", "dv")
         for f in ((name, ctypes.c_void_p), (f"{name}_stride_b", ctypes.c_int64),
                   (f"{name}_stride_h", ctypes.c_int64), (f"{name}_stride_s", ctypes.c_int64))] + [
        ("lse", ctypes.c_void_p),
        ("lse_stride_b", ctypes.c_int64), ("lse_stride_h", ctypes.c_int64),
        ("sm_scale", ctypes.c_float),
    ]


class EsaNaiveOpts(ctypes.Structure):
    _fields_ = [
        ("dropout_p", ctypes.c_float),
        ("seed", ctypes.c_uint64),
        ("weights", ctypes.c_void_p),
        ("weights_stride_b", ctypes.c_int64), ("weights_stride_h", ctypes.c_int64),
        ("weights_stride_s", ctypes.c_int64),
    ]


_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Loads libesa.so once and declares every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with "
            "`python elastic-sparse-attention_amd/build_lib.py` (hipcc, gfx950)")
    lib = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER
    st = ctypes.c_int32
    vp = ctypes.c_void_p
    lib.esa_status_string.restype = ctypes.c_char_p
    lib.esa_status_string.argtypes = [st]
    lib.esa_version.restype = ctypes.c_char_p
    lib.esa_version.argtypes = []
    lib.esa_layout_sizes.restype = st
    lib.esa_layout_sizes.argtypes = [P(EsaPattern), P(ctypes.c_int32), P(ctypes.c_int32),
                                     P(ctypes.c_int64), P(ctypes.c_size_t)]
    lib.esa_build_indices.restype = st
    lib.esa_build_indices.argtypes = [P(EsaPattern), ctypes.c_int32, ctypes.c_int32, vp, vp,
                                      ctypes.c_int32, vp]
    lib.esa_build_dense_mask.restype = st
    lib.esa_build_dense_mask.argtypes = [P(EsaPattern), ctypes.c_int32, ctypes.c_int32,
                                         ctypes.c_int32, vp, ctypes.c_int64, ctypes.c_int64, vp]
    lib.esa_build_layout.restype = st
    lib.esa_build_layout.argtypes = [P(EsaPattern), vp, vp, ctypes.c_int64, vp, ctypes.c_size_t,
                                     vp]
    lib.esa_plan_schedule.restype = st
    lib.esa_plan_schedule.argtypes = [P(EsaPattern), vp, ctypes.c_int32, ctypes.c_int32, vp,
                                      ctypes.c_int64, P(ctypes.c_int64)]
    lib.esa_elastic_fwd.restype = st
    lib.esa_elastic_fwd.argtypes = [P(EsaFwdArgs), P(EsaPattern), vp, vp, vp, vp, ctypes.c_int64,
                                    vp, ctypes.c_int64, vp]
    lib.esa_stage_masks_size.restype = st
    lib.esa_stage_masks_size.argtypes = [P(EsaPattern), vp, P(ctypes.c_int64)]
    lib.esa_build_stage_masks.restype = st
    lib.esa_build_stage_masks.argtypes = [P(EsaPattern), vp, vp, vp, vp, ctypes.c_int64, vp]
    lib.esa_elastic_fwd_band.restype = st
    lib.esa_elastic_fwd_band.argtypes = [P(EsaFwdArgs), P(EsaPattern), vp, vp]
    lib.esa_elastic_fwd_rows.restype = st
    lib.esa_elastic_fwd_rows.argtypes = [P(EsaFwdArgs), P(EsaPattern), vp, vp]
    lib.esa_sparse_fwd.restype = st
    lib.esa_sparse_fwd.argtypes = [P(EsaFwdArgs), vp, ctypes.c_int32, ctypes.c_int64,
                                   ctypes.c_int64, vp, ctypes.c_int32, ctypes.c_int64,
                                   ctypes.c_int64, ctypes.c_int32, vp]
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    lib.esa_plan_bwd.restype = st
    lib.esa_plan_bwd.argtypes = [P(EsaPattern), vp, vp, i32, i32, i32, vp, vp, vp, i64, vp, i64,
                                 P(i64), P(i64)]
    lib.esa_build_tile_masks.restype = st
    lib.esa_build_tile_masks.argtypes = [P(EsaPattern), vp, vp, vp, i32, vp, i64, vp]
    lib.esa_bwd_workspace_size.restype = st
    lib.esa_bwd_workspace_size.argtypes = [P(EsaBwdArgs), P(ctypes.c_size_t)]
    lib.esa_elastic_bwd.restype = st
    lib.esa_elastic_bwd.argtypes = [P(EsaBwdArgs), P(EsaPattern), vp, vp, vp, vp, i64, vp, vp, vp,
                                    vp, i64, vp, i64, vp, i64, vp, ctypes.c_size_t, vp]
    lib.esa_elastic_bwd_noalloc.restype = st
    lib.esa_elastic_bwd_noalloc.argtypes = [P(EsaBwdArgs), P(EsaPattern), vp, vp, vp, vp, i64, vp,
                                            vp, vp, vp, i64, vp, i64, vp, i64, vp]
    lib.esa_init_device.restype = st
    lib.esa_init_device.argtypes = [i32]
    lib.esa_bwd_noalloc_max_workspace.restype = ctypes.c_size_t
    lib.esa_bwd_noalloc_max_workspace.argtypes = []
    lib.esa_elastic_fwd_naive.restype = st
    lib.esa_elastic_fwd_naive.argtypes = [P(EsaFwdArgs), P(EsaPattern), vp, P(EsaNaiveOpts), vp]
    lib.esa_gather_bwd_workspace_size.restype = st
    lib.esa_gather_bwd_workspace_size.argtypes = [P(EsaBwdArgs), i32, P(ctypes.c_size_t)]
    lib.esa_sparse_bwd.restype = st
    lib.esa_sparse_bwd.argtypes = [P(EsaBwdArgs), vp, i32, i64, i64, vp, i32, i64, i64, i32, vp,
                                   ctypes.c_size_t, vp]
    lib.esa_elastic_bwd_rows.restype = st
    lib.esa_elastic_bwd_rows.argtypes = [P(EsaBwdArgs), P(EsaPattern), vp, ctypes.c_float,
                                         ctypes.c_uint64, vp, ctypes.c_size_t, vp]
    i32 = ctypes.c_int32
    lib.esa_reachability.restype = st
    lib.esa_reachability.argtypes = [i32, i32, i32, i32, i32, vp, vp, vp, vp]
    _lib = lib
    return lib


PROBE_EXPORTED = ("esa_probe_mfma_bf16", "esa_probe_l2_to_lds", "esa_probe_hbm_read",
                  "esa_probe_gather_to_lds", "esa_probe_gather_read", "esa_probe_lds_read")
_probe: Optional[ctypes.CDLL] = None


def load_probe() -> ctypes.CDLL:
    """Loads libesa_probe.so (include/esa_probe.h: the rate probes bench.py
    --peaks runs) once and declares its entry points."""
    global _probe
    if _probe is not None:
        return _probe
    if not os.path.exists(PROBE_LIB_PATH):
        raise RuntimeError(
            f"{PROBE_LIB_PATH} is missing: build it with "
            "`python elastic-sparse-attention_amd/build_lib.py` (hipcc, gfx950)")
    lib = ctypes.CDLL(PROBE_LIB_PATH)
    st, vp, i32, i64 = ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    lib.esa_probe_mfma_bf16.restype = st
    lib.esa_probe_mfma_bf16.argtypes = [i32, i32, ctypes.c_uint16, vp, i64, vp]
    lib.esa_probe_l2_to_lds.restype = st
    lib.esa_probe_l2_to_lds.argtypes = [vp, i64, i32, i32, i32, vp, i64, vp]
    lib.esa_probe_hbm_read.restype = st
    lib.esa_probe_hbm_read.argtypes = [vp, i64, i32, vp, i64, vp]
    lib.esa_probe_gather_to_lds.restype = st
    lib.esa_probe_gather_to_lds.argtypes = [vp, i64, vp, i64, i32, i32, vp, i64, vp]
    lib.esa_probe_gather_read.restype = st
    lib.esa_probe_gather_read.argtypes = [vp, i64, vp, i64, i32, vp, i64, vp]
    lib.esa_probe_lds_read.restype = st
    lib.esa_probe_lds_read.argtypes = [i32, i32, i32, vp, i64, vp]
    _probe = lib
    return lib


class EsaError(RuntimeError):
    """A HIP-side failure or a configuration the kernels do not cover."""


def check(status: int, what: str) -> None:
    """Maps an esa_status to a Python exception (argument errors -> ValueError)."""
    if status == ESA_OK:
        return
    msg = f"{what}: {load().esa_status_string(status).decode()} (esa_status {status})"
    if status in (ESA_ERR_NULL, ESA_ERR_SHAPE, ESA_ERR_DTYPE, ESA_ERR_ALIGN, ESA_ERR_CAPACITY):
        raise ValueError(msg)
    raise EsaError(msg)
