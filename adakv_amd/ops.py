"""Torch-facing, batched wrappers over the C-ABI of ``libadakv_amd.so``.

PyTorch supplies device memory and the current HIP stream; all computation is
in the HIP kernels.  Tensors must live on a ROCm device: there is no CPU path.

Layouts (head_dim contiguous, any other strides):
    q         [B, Hq, D]
    k, v      [B, Hkv, S, D]          (k and v share one stride set)
    centroid  [B, Hkv, max_blocks, D] (contiguous) -- or, for the minmax (Quest)
              estimator, [B, Hkv, max_blocks, 2*D]: per block the per-dimension
              max of its keys, then their min.  Every op that takes a summary
              reads its kind from its last dimension (D or 2*D); ``estimator=``
              states it explicitly.
    table     [B, Hq, T] int32, sel_lens [B, Hq] int32
    seq_lens  [B] int32 on the device, or None (= every sequence holds S tokens)
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _capi as C

_DTYPES = {torch.float32: C.ADAKV_F32, torch.float16: C.ADAKV_F16, torch.bfloat16: C.ADAKV_BF16}
_POLICIES = {"fixed": C.POLICY_FIXED, "adaptive": C.POLICY_ADAPTIVE,
             "adaptive_nucleus": C.POLICY_NUCLEUS}


@dataclass(frozen=True)
class BudgetParams:
    """``plan_selection`` keyword arguments (adakv/attention.py:149-162)."""
    avg_budget: float = 8
    k_min: int = 2
    k_max: int = 64
    n_sink_blocks: int = 1
    n_local_blocks: int = 4
    c_min: int = 1
    temperature: float = 1.0
    budget_policy: str = "adaptive"
    nucleus_p: float = 0.9

    def to_c(self) -> C.Budget:
        if self.budget_policy not in _POLICIES:
            raise ValueError(f"unknown budget_policy: {self.budget_policy!r}")
        return C.Budget(float(self.avg_budget), int(self.k_min), int(self.k_max),
                        int(self.n_sink_blocks), int(self.n_local_blocks), int(self.c_min),
                        float(self.temperature), _POLICIES[self.budget_policy], float(self.nucleus_p))


def _dt(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype} (float32, float16, bfloat16)") from None


def _on_device(*ts) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "AdaKV runs only as HIP kernels on a ROCm device; got a CPU tensor "
                "(the NumPy oracle under oracle/ is the CPU reference, for tests)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


_WORKSPACES: dict = {}


def workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """Zero-initialised scratch per (device, stream), grown on demand.  The
    kernels leave its counters zeroed, so it is reused without re-clearing."""
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(int(nbytes), 1 << 16), dtype=torch.uint8, device=dev)
        _WORKSPACES[key] = ws
    return ws


def _check_last(t: torch.Tensor, name: str) -> None:
    if t.stride(-1) != 1:
        raise ValueError(f"{name}: head_dim must be the contiguous axis")


def _q(q: torch.Tensor) -> C.Query:
    if q.dim() != 3:
        raise ValueError(f"q must be [B, Hq, D], got {tuple(q.shape)}")
    _check_last(q, "q")
    return C.Query(q.data_ptr(), _dt(q), q.stride(0), q.stride(1))


def _out(o: torch.Tensor) -> C.Output:
    _check_last(o, "out")
    return C.Output(o.data_ptr(), _dt(o), o.stride(0), o.stride(1))


def _kv(k: torch.Tensor, v: torch.Tensor | None) -> C.KV:
    if k.dim() != 4:
        raise ValueError(f"k must be [B, Hkv, S, D], got {tuple(k.shape)}")
    _check_last(k, "k")
    if v is not None:
        if v.shape != k.shape or v.dtype != k.dtype:
            raise ValueError("k and v must have the same shape and dtype")
        if v.stride() != k.stride():
            raise ValueError("k and v must share one stride layout")
    return C.KV(k.data_ptr(), v.data_ptr() if v is not None else None, _dt(k),
                k.stride(0), k.stride(1), k.stride(2))


_ESTIMATORS = {"centroid": C.SUMMARY_CENTROID, "minmax": C.SUMMARY_MINMAX}


def summary_kind(c: torch.Tensor, head_dim: int, estimator: str | None = None) -> str:
    """The estimator a summary tensor serves: its last dimension is head_dim
    (centroid) or 2 * head_dim (minmax); ``estimator`` must agree when given."""
    if estimator is not None and estimator not in _ESTIMATORS:
        raise ValueError(f"unknown estimator: {estimator!r}")
    last = c.shape[-1]
    kind = "centroid" if last == head_dim else "minmax" if last == 2 * head_dim else None
    if kind is None:
        raise ValueError(f"summary rows hold {last} elements; expected head_dim ({head_dim}) for "
                         f"centroids or 2*head_dim ({2 * head_dim}) for minmax bounds")
    if estimator is not None and estimator != kind:
        if estimator == "minmax":
            raise ValueError("minmax estimator needs minmax summaries [.., 2*head_dim] "
                             "(AdaKVCache(estimator='minmax'))")
        raise ValueError(f"estimator {estimator!r} does not match {kind} summaries")
    return kind


def _centroid(c: torch.Tensor, head_dim: int, estimator: str | None = None) -> C.Centroid:
    if c.dim() != 4 or not c.is_contiguous():
        raise ValueError("centroid must be a contiguous [B, Hkv, max_blocks, D or 2*D] tensor")
    return C.Centroid(c.data_ptr(), _dt(c), _ESTIMATORS[summary_kind(c, head_dim, estimator)])


def geometry(B, Hq, Hkv, D, block_size, max_seq_len, max_blocks) -> C.Geometry:
    if Hkv <= 0 or Hq % Hkv:
        raise ValueError(f"n_q_heads ({Hq}) must be a multiple of n_kv_heads ({Hkv})")
    return C.Geometry(int(B), int(Hq), int(Hkv), int(D), int(block_size), int(max_seq_len),
                      int(max_blocks))


def _seq_lens(seq_lens, dev):
    if seq_lens is None:
        return None
    if seq_lens.dtype != torch.int32 or seq_lens.device != dev or not seq_lens.is_contiguous():
        raise ValueError("seq_lens must be a contiguous int32 tensor on the same device")
    return seq_lens


def n_blocks(seq_len: int, block_size: int) -> int:
    return -(-int(seq_len) // int(block_size))


# ---------------------------------------------------------------------------
def centroid_build(k: torch.Tensor, block_size: int, seq_lens=None, centroid=None,
                   centroid_dtype=None, max_blocks=None, estimator: str | None = None) -> torch.Tensor:
    """Block summaries of k [B, Hkv, S, D]: centroids [B, Hkv, max_blocks, D]
    (adakv/estimator.py:27-48) or, with ``estimator="minmax"`` (or a given
    ``centroid`` tensor of rows 2*D), the per-dimension [max | min] bounds
    [B, Hkv, max_blocks, 2*D] (adakv/estimator.py:50-57).  Rows past a
    sequence's last block are left as they were (zeros for a new tensor)."""
    dev = _on_device(k, centroid, seq_lens)
    B, Hkv, S, D = k.shape
    nb = n_blocks(S, block_size)
    if centroid is None:
        est = estimator or "centroid"
        if est not in _ESTIMATORS:
            raise ValueError(f"unknown estimator kind: {est!r}")
        cdt = centroid_dtype or (torch.float32 if k.dtype == torch.float32 else k.dtype)
        row = 2 * D if est == "minmax" else D
        centroid = torch.zeros(B, Hkv, max(max_blocks or nb, nb), row, dtype=cdt, device=dev)
    g = geometry(B, Hkv, Hkv, D, block_size, S, centroid.shape[2])
    C.check(C.load().adakv_centroid_build(ctypes.byref(g), ctypes.byref(_kv(k, None)),
                                          _ptr(_seq_lens(seq_lens, dev)),
                                          ctypes.byref(_centroid(centroid, D, estimator)), _stream(dev)),
            "centroid_build")
    return centroid


def centroid_append(k: torch.Tensor, centroid: torch.Tensor, block_size: int, n_new: int = 1,
                    seq_lens=None) -> torch.Tensor:
    """Refresh, in place, the summaries (centroids or minmax bounds) of the
    blocks holding the newest ``n_new`` tokens of every sequence
    (adakv/runtime.py:43-60)."""
    dev = _on_device(k, centroid, seq_lens)
    B, Hkv, S, D = k.shape
    g = geometry(B, Hkv, Hkv, D, block_size, S, centroid.shape[2])
    C.check(C.load().adakv_centroid_append(ctypes.byref(g), ctypes.byref(_kv(k, None)),
                                           _ptr(_seq_lens(seq_lens, dev)), int(n_new),
                                           ctypes.byref(_centroid(centroid, D)), _stream(dev)),
            "centroid_append")
    return centroid


def block_scores(q: torch.Tensor, centroid: torch.Tensor, block_size: int, seq_len=None,
                 seq_lens=None, out=None, estimator: str | None = None) -> torch.Tensor:
    """Score of every block, fp32 [B, Hq, max_blocks]: q . centroid
    (adakv/estimator.py:62-74) or, for minmax summaries, the Quest bound
    max(q,0) . kmax + min(q,0) . kmin (adakv/estimator.py:76-79)."""
    dev = _on_device(q, centroid, seq_lens, out)
    B, Hq, D = q.shape
    _, Hkv, maxb, _ = centroid.shape
    S = int(seq_len) if seq_len is not None else maxb * block_size
    g = geometry(B, Hq, Hkv, D, block_size, S, maxb)
    if out is None:
        out = torch.zeros(B, Hq, maxb, dtype=torch.float32, device=dev)
    if out.dtype != torch.float32 or not out.is_contiguous() or out.shape[:2] != (B, Hq):
        raise ValueError("scores must be a contiguous fp32 [B, Hq, pitch] tensor")
    C.check(C.load().adakv_block_scores(ctypes.byref(g), ctypes.byref(_q(q)),
                                        ctypes.byref(_centroid(centroid, D, estimator)),
                                        _ptr(_seq_lens(seq_lens, dev)), _ptr(out), out.shape[2],
                                        _stream(dev)), "block_scores")
    return out


def table_width(B, Hq, Hkv, D, block_size, max_seq_len, max_blocks, budget: BudgetParams) -> int:
    g = geometry(B, Hq, Hkv, D, block_size, max_seq_len, max_blocks)
    w = C.load().adakv_table_width(ctypes.byref(g), ctypes.byref(budget.to_c()))
    if w < 1:
        raise ValueError("invalid geometry or budget")
    return int(w)


def plan(q: torch.Tensor, centroid: torch.Tensor, block_size: int, budget: BudgetParams,
         seq_len: int | None = None, seq_lens=None, table=None, sel_lens=None,
         estimator: str | None = None):
    """Scores + budget + selection (adakv/attention.py:149-247).

    Returns (table [B, Hq, T] int32, sel_lens [B, Hq] int32); the first
    sel_lens[b, h] entries of a row are the selected blocks (forced blocks in
    ascending order, then content blocks by descending score)."""
    dev = _on_device(q, centroid, seq_lens)
    B, Hq, D = q.shape
    _, Hkv, maxb, _ = centroid.shape
    S = int(seq_len) if seq_len is not None else maxb * block_size
    g = geometry(B, Hq, Hkv, D, block_size, S, maxb)
    cb = budget.to_c()
    T = C.load().adakv_table_width(ctypes.byref(g), ctypes.byref(cb))
    if T < 1:
        C.check(C.ADAKV_ERR_SHAPE, "plan")
    if table is None:
        table = torch.empty(B, Hq, T, dtype=torch.int32, device=dev)
    if sel_lens is None:
        sel_lens = torch.empty(B, Hq, dtype=torch.int32, device=dev)
    if not (table.is_contiguous() and sel_lens.is_contiguous()) or table.dtype != torch.int32 \
            or sel_lens.dtype != torch.int32:
        raise ValueError("table / sel_lens must be contiguous int32")
    nbytes = C.load().adakv_workspace_bytes(ctypes.byref(g), table.shape[-1])
    ws = workspace(dev, nbytes)
    sel = C.Selection(table.data_ptr(), table.shape[-1], sel_lens.data_ptr())
    C.check(C.load().adakv_plan(ctypes.byref(g), ctypes.byref(_q(q)),
                                ctypes.byref(_centroid(centroid, D, estimator)),
                                _ptr(_seq_lens(seq_lens, dev)), ctypes.byref(cb), ctypes.byref(sel),
                                _ptr(ws), ws.numel(), _stream(dev)), "plan")
    return table, sel_lens


def sparse_decode(q, k, v, table, sel_lens, block_size: int, sm_scale=None, seq_lens=None,
                  out=None):
    """Attention over exactly the listed blocks
    (adakv/kernels/block_sparse_decode.py:103-135).  Output dtype = q dtype."""
    dev = _on_device(q, k, v, table, sel_lens, seq_lens, out)
    B, Hq, D = q.shape
    _, Hkv, S, _ = k.shape
    if table.dim() != 3 or table.shape[:2] != (B, Hq) or sel_lens.shape != (B, Hq):
        raise ValueError("table must be [B, Hq, T] and sel_lens [B, Hq]")
    if table.dtype != torch.int32 or sel_lens.dtype != torch.int32:
        raise ValueError("table and sel_lens must be int32")
    if not (table.is_contiguous() and sel_lens.is_contiguous()):
        raise ValueError("table and sel_lens must be contiguous")
    sm_scale = (1.0 / math.sqrt(D)) if sm_scale is None else float(sm_scale)
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q.dtype, device=dev)
    g = geometry(B, Hq, Hkv, D, block_size, S, n_blocks(S, block_size))
    T = table.shape[-1]
    nbytes = C.load().adakv_workspace_bytes(ctypes.byref(g), T)
    ws = workspace(dev, nbytes)
    sel = C.Selection(table.data_ptr(), T, sel_lens.data_ptr())
    C.check(C.load().adakv_sparse_decode(ctypes.byref(g), ctypes.byref(_q(q)), ctypes.byref(_kv(k, v)),
                                         _ptr(_seq_lens(seq_lens, dev)), ctypes.byref(sel),
                                         ctypes.c_float(sm_scale), ctypes.byref(_out(out)), _ptr(ws),
                                         ws.numel(), _stream(dev)), "sparse_decode")
    return out


def decode_fused(q, k, v, centroid, block_size: int, budget: BudgetParams, seq_lens=None,
                 append_new: int = 0, sm_scale=None, out=None, return_selection=False,
                 estimator: str | None = None):
    """One decode step: optional summary append, plan, sparse decode
    (adakv/attention.py:250-268).  ``centroid`` holds centroids or minmax
    bounds (the estimator, by its row length)."""
    dev = _on_device(q, k, v, centroid, seq_lens, out)
    B, Hq, D = q.shape
    _, Hkv, S, _ = k.shape
    maxb = centroid.shape[2]
    g = geometry(B, Hq, Hkv, D, block_size, S, maxb)
    cb = budget.to_c()
    T = C.load().adakv_table_width(ctypes.byref(g), ctypes.byref(cb))
    if T < 1:
        C.check(C.ADAKV_ERR_SHAPE, "decode_fused")
    sm_scale = (1.0 / math.sqrt(D)) if sm_scale is None else float(sm_scale)
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q.dtype, device=dev)
    table = lens = None
    sel_ref = None
    if return_selection:
        table = torch.empty(B, Hq, T, dtype=torch.int32, device=dev)
        lens = torch.empty(B, Hq, dtype=torch.int32, device=dev)
        sel_ref = ctypes.byref(C.Selection(table.data_ptr(), T, lens.data_ptr()))
    nbytes = C.load().adakv_workspace_bytes(ctypes.byref(g), T)
    ws = workspace(dev, nbytes)
    C.check(C.load().adakv_decode_fused(ctypes.byref(g), ctypes.byref(_q(q)), ctypes.byref(_kv(k, v)),
                                        ctypes.byref(_centroid(centroid, D, estimator)),
                                        _ptr(_seq_lens(seq_lens, dev)), ctypes.byref(cb), sel_ref,
                                        int(append_new), ctypes.c_float(sm_scale),
                                        ctypes.byref(_out(out)), _ptr(ws), ws.numel(), _stream(dev)),
            "decode_fused")
    if return_selection:
        return out, table, lens
    return out


def decode_fused_scan(q, k, v, centroid, block_size: int, budget: BudgetParams, seq_lens=None,
                      append_new: int = 0, estimator: str | None = None):
    """The first of decode_fused's two launches, alone and as the step issues
    it: summary append, block scores and their softmax records (left in the
    workspace).  For timing the step's launches separately."""
    dev = _on_device(q, k, v, centroid, seq_lens)
    B, Hq, D = q.shape
    _, Hkv, S, _ = k.shape
    g = geometry(B, Hq, Hkv, D, block_size, S, centroid.shape[2])
    cb = budget.to_c()
    T = C.load().adakv_table_width(ctypes.byref(g), ctypes.byref(cb))
    if T < 1:
        C.check(C.ADAKV_ERR_SHAPE, "decode_fused_scan")
    ws = workspace(dev, C.load().adakv_workspace_bytes(ctypes.byref(g), T))
    C.check(C.load().adakv_decode_fused_scan(ctypes.byref(g), ctypes.byref(_q(q)), ctypes.byref(_kv(k, v)),
                                             ctypes.byref(_centroid(centroid, D, estimator)),
                                             _ptr(_seq_lens(seq_lens, dev)), ctypes.byref(cb), int(append_new),
                                             _ptr(ws), ws.numel(), _stream(dev)),
            "decode_fused_scan")


def dense_decode(q, k, v, sm_scale=None, seq_lens=None, out=None):
    """Dense split-K flash-decode over every token (bench_decode_latency.py:40-53)."""
    dev = _on_device(q, k, v, seq_lens, out)
    B, Hq, D = q.shape
    _, Hkv, S, _ = k.shape
    sm_scale = (1.0 / math.sqrt(D)) if sm_scale is None else float(sm_scale)
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q.dtype, device=dev)
    g = geometry(B, Hq, Hkv, D, 16, S, n_blocks(S, 16))
    nbytes = C.load().adakv_workspace_bytes(ctypes.byref(g), 1)
    ws = workspace(dev, nbytes)
    C.check(C.load().adakv_dense_decode(ctypes.byref(g), ctypes.byref(_q(q)), ctypes.byref(_kv(k, v)),
                                        _ptr(_seq_lens(seq_lens, dev)), ctypes.c_float(sm_scale),
                                        ctypes.byref(_out(out)), _ptr(ws), ws.numel(), _stream(dev)),
            "dense_decode")
    return out
