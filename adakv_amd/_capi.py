"""ctypes binding of ``libadakv_amd.so`` (declared in ``include/adakv_amd.h``).

Only plain pointers, sizes and a stream handle cross this boundary.  The
library is loaded lazily; every entry point raises if it is missing, so there
is no silent CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

from . import build as _build

c_int32 = ctypes.c_int32
c_int64 = ctypes.c_int64
c_void_p = ctypes.c_void_p

ADAKV_OK = 0
ADAKV_ERR_NULL = 1
ADAKV_ERR_SHAPE = 2
ADAKV_ERR_DTYPE = 3
ADAKV_ERR_UNSUPPORTED = 4
ADAKV_ERR_WORKSPACE = 5
ADAKV_ERR_LAUNCH = 6
ADAKV_ERR_VALUE = 7
ADAKV_ERR_SCRATCH = 8
NOALLOC_SCRATCH_BYTES = 16 << 20

ADAKV_F32, ADAKV_F16, ADAKV_BF16 = 0, 1, 2
POLICY_FIXED, POLICY_ADAPTIVE, POLICY_NUCLEUS = 0, 1, 2
SUMMARY_CENTROID, SUMMARY_MINMAX = 0, 1
ABI_VERSION = 6


class Geometry(ctypes.Structure):
    _fields_ = [("batch", c_int32), ("n_q_heads", c_int32), ("n_kv_heads", c_int32),
                ("head_dim", c_int32), ("block_size", c_int32), ("max_seq_len", c_int32),
                ("max_blocks", c_int32)]


class Query(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("dtype", c_int32), ("stride_b", c_int64),
                ("stride_h", c_int64)]


class Output(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("dtype", c_int32), ("stride_b", c_int64),
                ("stride_h", c_int64)]


class KV(ctypes.Structure):
    _fields_ = [("k", c_void_p), ("v", c_void_p), ("dtype", c_int32), ("stride_b", c_int64),
                ("stride_h", c_int64), ("stride_s", c_int64)]


class Centroid(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("dtype", c_int32), ("kind", c_int32)]


class Budget(ctypes.Structure):
    _fields_ = [("avg_budget", ctypes.c_double), ("k_min", c_int32), ("k_max", c_int32),
                ("n_sink_blocks", c_int32), ("n_local_blocks", c_int32), ("c_min", c_int32),
                ("temperature", ctypes.c_double), ("policy", c_int32), ("nucleus_p", ctypes.c_double)]


class Selection(ctypes.Structure):
    _fields_ = [("block_table", c_void_p), ("table_width", c_int32), ("sel_lens", c_void_p)]


class Prompt(ctypes.Structure):
    _fields_ = [("q", c_void_p), ("k", c_void_p), ("dtype", c_int32), ("n_q_heads", c_int32),
                ("n_kv_heads", c_int32), ("head_dim", c_int32), ("n_tokens", c_int32),
                ("q_stride_h", ctypes.c_int64), ("q_stride_s", ctypes.c_int64),
                ("k_stride_h", ctypes.c_int64), ("k_stride_s", ctypes.c_int64)]


P = ctypes.POINTER
SIGNATURES = {
    "adakv_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "adakv_abi_version": (ctypes.c_int, []),
    "adakv_table_width": (c_int32, [P(Geometry), P(Budget)]),
    "adakv_workspace_bytes": (ctypes.c_size_t, [P(Geometry), c_int32]),
    "adakv_centroid_build": (ctypes.c_int, [P(Geometry), P(KV), c_void_p, P(Centroid), c_void_p]),
    "adakv_centroid_append": (ctypes.c_int, [P(Geometry), P(KV), c_void_p, c_int32, P(Centroid),
                                             c_void_p]),
    "adakv_block_scores": (ctypes.c_int, [P(Geometry), P(Query), P(Centroid), c_void_p, c_void_p,
                                          c_int32, c_void_p]),
    "adakv_plan": (ctypes.c_int, [P(Geometry), P(Query), P(Centroid), c_void_p, P(Budget),
                                  P(Selection), c_void_p, ctypes.c_size_t, c_void_p]),
    "adakv_sparse_decode": (ctypes.c_int, [P(Geometry), P(Query), P(KV), c_void_p, P(Selection),
                                           ctypes.c_float, P(Output), c_void_p, ctypes.c_size_t,
                                           c_void_p]),
    "adakv_decode_fused": (ctypes.c_int, [P(Geometry), P(Query), P(KV), P(Centroid), c_void_p,
                                          P(Budget), P(Selection), c_int32, ctypes.c_float,
                                          P(Output), c_void_p, ctypes.c_size_t, c_void_p]),
    "adakv_decode_fused_scan": (ctypes.c_int, [P(Geometry), P(Query), P(KV), P(Centroid), c_void_p,
                                               P(Budget), c_int32, c_void_p, ctypes.c_size_t, c_void_p]),
    "adakv_decode_fused_noalloc": (ctypes.c_int, [P(Geometry), P(Query), P(KV), P(Centroid), c_void_p,
                                                  P(Budget), P(Selection), c_int32, ctypes.c_float,
                                                  P(Output), c_void_p]),
    "adakv_dense_decode": (ctypes.c_int, [P(Geometry), P(Query), P(KV), c_void_p, ctypes.c_float,
                                          P(Output), c_void_p, ctypes.c_size_t, c_void_p]),
    "adakv_importance_workspace_bytes": (ctypes.c_size_t, [P(Prompt), c_int32]),
    "adakv_key_importance": (ctypes.c_int, [P(Prompt), c_int32, ctypes.c_float, c_void_p, c_int32,
                                            c_void_p, ctypes.c_size_t, c_void_p]),
    "adakv_importance_pool": (ctypes.c_int, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32,
                                             c_void_p]),
    "adakv_retain_blocks": (ctypes.c_int, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                                           c_int32, c_int32, c_void_p, c_int32, P(Selection), c_void_p]),
    "adakv_frozen_table": (ctypes.c_int, [P(Selection), c_int32, c_int32, c_int32, c_int32, c_int32,
                                          P(Selection), c_void_p]),
    "adakv_mask_table": (ctypes.c_int, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                                        P(Selection), c_void_p]),
}

_LIB = None
_LOAD_ERROR: str | None = None


def lib_path() -> str:
    return os.environ.get("ADAKV_LIB", _build.lib_path())


def load():
    """Load and bind the library (cached).  Raises RuntimeError when absent."""
    global _LIB, _LOAD_ERROR
    if _LIB is not None:
        return _LIB
    path = lib_path()
    if not os.path.exists(path):
        _LOAD_ERROR = f"{path} not built (run `python -m adakv_amd.build`)"
        raise RuntimeError(f"AdaKV HIP library missing: {_LOAD_ERROR}")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.adakv_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {lib.adakv_abi_version()} != {ABI_VERSION}")
    _LIB = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


class AdaKVError(RuntimeError):
    """A non-argument failure reported by the library (workspace, launch)."""


def check(status: int, what: str) -> None:
    """Map a C status to the reference's error behaviour: argument problems are
    ValueError (adakv/estimator.py:59, budget.py:42, attention.py:192-226),
    runtime failures AdaKVError."""
    if status == ADAKV_OK:
        return
    msg = f"{what}: {load().adakv_status_string(status).decode()} (status {status})"
    if status in (ADAKV_ERR_NULL, ADAKV_ERR_SHAPE, ADAKV_ERR_DTYPE, ADAKV_ERR_VALUE, ADAKV_ERR_SCRATCH,
                  ADAKV_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise AdaKVError(msg)
