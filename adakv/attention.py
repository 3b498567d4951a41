"""Runtime attention module: AdaKV cache, selection planner, decode step
(adakv/attention.py).

The planner and the decode run as HIP kernels (``libadakv_amd.so``) on the
current stream.  ``plan_selection`` returns the reference's table width,
``max(sel_lens)``, which takes one device->host read of the counts as the
reference's does (adakv/attention.py:242); the decode step
(``adakv_decode_attention``, ``adakv_decode_step``, the HF hook) plans and
decodes in one C call at the static width (``adakv_table_width``) with no
host synchronisation.  Entries of a row past ``sel_lens[h]`` are
further-ranked candidates or -1 and are never read.

The instrumentation (budget trace, recall) is kept with the reference's
names; it reads the selection back to the host only while it is switched on.
"""
from __future__ import annotations

import math

import torch

from adakv_amd import ops

# --- realised-budget instrumentation (adakv/attention.py:24-45) -------------
_BUDGET_TRACE = None


def reset_budget_trace():
    """Start (or restart) recording the realised mean blocks/head per decode step."""
    global _BUDGET_TRACE
    _BUDGET_TRACE = []


def get_budget_trace():
    """Per-step mean blocks/head recorded since the last reset."""
    return list(_BUDGET_TRACE) if _BUDGET_TRACE is not None else []


def stop_budget_trace():
    """Disable recording."""
    global _BUDGET_TRACE
    _BUDGET_TRACE = None


# --- selection-recall instrumentation (adakv/attention.py:48-88) --------------
_RECALL_TARGET = None
_RECALL_HITS = 0
_RECALL_TOTAL = 0


def set_recall_target(block_ids):
    """Begin recording coverage of these block indices; resets the counters."""
    global _RECALL_TARGET, _RECALL_HITS, _RECALL_TOTAL
    _RECALL_TARGET = {int(b) for b in block_ids}
    _RECALL_HITS = 0
    _RECALL_TOTAL = 0


def get_recall():
    """Fraction of (decode step, target block) pairs selected by at least one head."""
    return (_RECALL_HITS / _RECALL_TOTAL) if _RECALL_TOTAL else float("nan")


def clear_recall_target():
    global _RECALL_TARGET
    _RECALL_TARGET = None


def _record_recall(block_table, sel_lens, nb):
    global _RECALL_HITS, _RECALL_TOTAL
    bt = block_table.reshape(-1, block_table.shape[-1]).cpu()
    sl = sel_lens.reshape(-1).cpu()
    chosen = set()
    for h in range(bt.shape[0]):
        chosen.update(int(x) for x in bt[h, : int(sl[h])].tolist())
    for b in _RECALL_TARGET:
        if 0 <= b < nb:
            _RECALL_TOTAL += 1
            _RECALL_HITS += int(b in chosen)


def record_selection(block_table, sel_lens, nb):
    """Record realised budget and target coverage for one step, if either
    instrument is on (adakv/attention.py:91-103)."""
    if _BUDGET_TRACE is not None:
        _BUDGET_TRACE.append(float(sel_lens.float().mean().item()))
    if _RECALL_TARGET is not None:
        _record_recall(block_table, sel_lens, nb)


def instrumentation_active() -> bool:
    return _BUDGET_TRACE is not None or _RECALL_TARGET is not None


class AdaKVCache:
    """Full KV cache plus block summaries resident in HBM (adakv/attention.py:106-146).

    ``k``/``v`` are ``[n_kv_heads, S, D]`` views of the current length;
    ``centroid`` is ``[n_kv_heads, n_blocks, D]``.  With ``estimator="minmax"``
    the cache also holds Quest's per-block key bounds (attention.py:131-138),
    stored as one ``[n_kv_heads, n_blocks, 2*D]`` buffer of rows [max | min];
    ``kmax`` and ``kmin`` are ``[n_kv_heads, n_blocks, D]`` views of it.
    Decode appends write into preallocated storage and refresh only the
    trailing blocks' summaries.  ``centroid_dtype`` (the summaries' dtype)
    defaults to the key dtype (fp32 keys: fp32); minmax bounds are kept in
    the key dtype or fp32, where they are exact.
    """

    def __init__(self, block_size: int, estimator: str = "centroid", centroid_dtype=None):
        if estimator not in ("centroid", "minmax"):
            raise ValueError(f"unknown estimator kind: {estimator!r}")
        self.block_size = int(block_size)
        self.estimator = estimator
        self.centroid_dtype = centroid_dtype
        self.k = None
        self.v = None
        self._kbuf = None
        self._vbuf = None
        self._cbuf = None          # [1, Hkv, capacity_blocks, D]
        self._mbuf = None          # [1, Hkv, capacity_blocks, 2*D] (minmax only)

    @property
    def seq_len(self) -> int:
        return 0 if self.k is None else int(self.k.shape[1])

    @property
    def n_blocks(self) -> int:
        return ops.n_blocks(self.seq_len, self.block_size)

    @property
    def centroid(self):
        if self._cbuf is None:
            return None
        return self._cbuf[0, :, : self.n_blocks]

    @property
    def kmax(self):
        """Per-block per-dimension key maxima [Hkv, n_blocks, D] (minmax caches)."""
        if self._mbuf is None:
            return None
        return self._mbuf[0, :, : self.n_blocks, : self._mbuf.shape[3] // 2]

    @property
    def kmin(self):
        """Per-block per-dimension key minima [Hkv, n_blocks, D] (minmax caches)."""
        if self._mbuf is None:
            return None
        return self._mbuf[0, :, : self.n_blocks, self._mbuf.shape[3] // 2:]

    def summary(self, estimator: str):
        """The [1, Hkv, capacity_blocks, row] summary buffer an estimator scores."""
        if estimator == "minmax":
            if self._mbuf is None:
                raise ValueError("minmax estimator needs AdaKVCache(estimator='minmax')")
            return self._mbuf
        if estimator != "centroid":
            raise ValueError(f"unknown estimator: {estimator!r}")
        return self._cbuf

    def append_prefill(self, k, v):
        """Store the prefill KV and build every block summary. k, v: [Hkv, S, D]."""
        self.k, self.v = k, v
        self._kbuf = self._vbuf = None
        Hkv, S, D = k.shape
        nb = ops.n_blocks(S, self.block_size)
        cdt = self.centroid_dtype or (torch.float32 if k.dtype == torch.float32 else k.dtype)
        cap = nb + max(64, nb // 8)
        self._cbuf = torch.zeros(1, Hkv, cap, D, dtype=cdt, device=k.device)
        ops.centroid_build(k.unsqueeze(0), self.block_size, centroid=self._cbuf)
        self._mbuf = None
        if self.estimator == "minmax":
            mdt = cdt if cdt in (k.dtype, torch.float32) else torch.float32
            self._mbuf = torch.zeros(1, Hkv, cap, 2 * D, dtype=mdt, device=k.device)
            ops.centroid_build(k.unsqueeze(0), self.block_size, centroid=self._mbuf)
        return self

    @staticmethod
    def _grown(buf, nb):
        if nb <= buf.shape[2]:
            return buf
        grown = torch.zeros(1, buf.shape[1], nb + max(64, nb // 8), buf.shape[3], dtype=buf.dtype,
                            device=buf.device)
        grown[:, :, : buf.shape[2]].copy_(buf)
        return grown

    def _grow_kv(self, need: int):
        Hkv, S, D = self.k.shape
        cap = max(need, S + S // 4 + 1024)
        kb = torch.empty(Hkv, cap, D, dtype=self.k.dtype, device=self.k.device)
        vb = torch.empty_like(kb)
        kb[:, :S].copy_(self.k)
        vb[:, :S].copy_(self.v)
        self._kbuf, self._vbuf = kb, vb

    def append_decode(self, k_t, v_t):
        """Append decoded tokens' KV (k_t, v_t: [Hkv, n, D]) and refresh the
        affected summaries in O(block_size * D) per KV head (adakv/runtime.py:43-60)."""
        S, n = self.seq_len, int(k_t.shape[1])
        if self._kbuf is None or S + n > self._kbuf.shape[1]:
            self._grow_kv(S + n)
        self._kbuf[:, S:S + n].copy_(k_t)
        self._vbuf[:, S:S + n].copy_(v_t)
        self.k = self._kbuf[:, : S + n]
        self.v = self._vbuf[:, : S + n]
        nb = ops.n_blocks(S + n, self.block_size)
        self._cbuf = self._grown(self._cbuf, nb)
        ops.centroid_append(self.k.unsqueeze(0), self._cbuf, self.block_size, n_new=n)
        if self._mbuf is not None:
            self._mbuf = self._grown(self._mbuf, nb)
            ops.centroid_append(self.k.unsqueeze(0), self._mbuf, self.block_size, n_new=n)
        return self


def _budget(avg_budget, k_min, k_max, n_sink_blocks, n_local_blocks, temperature, budget_policy,
            c_min, nucleus_p=0.9):
    return ops.BudgetParams(avg_budget=avg_budget, k_min=k_min, k_max=k_max,
                            n_sink_blocks=n_sink_blocks, n_local_blocks=n_local_blocks,
                            c_min=c_min, temperature=temperature, budget_policy=budget_policy,
                            nucleus_p=nucleus_p)


def _validate(cache, estimator, budget_policy):
    """The summary buffer the estimator scores (adakv/attention.py:185-198 errors)."""
    if estimator == "minmax" and (cache.kmin is None or cache.kmax is None):
        raise ValueError("minmax estimator needs AdaKVCache(estimator='minmax')")
    if estimator not in ("centroid", "minmax"):
        raise ValueError(f"unknown estimator: {estimator!r}")
    if budget_policy not in ("fixed", "adaptive", "adaptive_nucleus"):
        raise ValueError(f"unknown budget_policy: {budget_policy!r}")
    return cache.summary(estimator)


def plan_selection(q, cache: AdaKVCache, avg_budget, k_min: int = 2, k_max: int = 64,
                   n_sink_blocks: int = 1, n_local_blocks: int = 4, temperature: float = 1.0,
                   estimator: str = "centroid", budget_policy: str = "adaptive", c_min: int = 1,
                   nucleus_p: float = 0.9):
    """Score blocks, allocate the per-head budget, select blocks
    (adakv/attention.py:149-247).  q: [Hq, D].

    Returns (block_table int32 [Hq, max(sel_lens)], sel_lens int32 [Hq]);
    rows hold the forced sink/local blocks, then content blocks by descending
    score.  The width is the largest count, as the reference returns it
    (adakv/attention.py:242-244): one read of the counts to the host.
    """
    summ = _validate(cache, estimator, budget_policy)
    budget = _budget(avg_budget, k_min, k_max, n_sink_blocks, n_local_blocks, temperature,
                     budget_policy, c_min, nucleus_p)
    table, lens = ops.plan(q.unsqueeze(0), summ, cache.block_size, budget,
                           seq_len=cache.seq_len, estimator=estimator)
    block_table, sel_lens = table[0], lens[0]
    max_sel = int(sel_lens.max().item()) if sel_lens.numel() else 0
    block_table = block_table[:, :max_sel].contiguous()
    record_selection(block_table, sel_lens, cache.n_blocks)
    return block_table, sel_lens


def adakv_decode_attention(q, cache: AdaKVCache, avg_budget, k_min: int = 2, k_max: int = 64,
                           n_sink_blocks: int = 1, n_local_blocks: int = 4,
                           temperature: float = 1.0, estimator: str = "centroid",
                           budget_policy: str = "adaptive", c_min: int = 1, nucleus_p: float = 0.9):
    """One AdaKV decode step: plan + sparse decode in one C call (two or three
    kernels, no host sync).  q: [Hq, D] -> [Hq, D] (adakv/attention.py:250-268;
    the estimator / policy keywords are plan_selection's)."""
    summ = _validate(cache, estimator, budget_policy)
    budget = _budget(avg_budget, k_min, k_max, n_sink_blocks, n_local_blocks, temperature,
                     budget_policy, c_min, nucleus_p)
    D = q.shape[-1]
    res = ops.decode_fused(q.unsqueeze(0), cache.k.unsqueeze(0), cache.v.unsqueeze(0), summ,
                           cache.block_size, budget, sm_scale=1.0 / math.sqrt(D),
                           return_selection=instrumentation_active(), estimator=estimator)
    if instrumentation_active():
        out, table, lens = res
        record_selection(table[0], lens[0], cache.n_blocks)
        return out[0]
    return res[0]
