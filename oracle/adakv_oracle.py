"""CPU oracle for the AdaKV decode hot path -- TEST INFRASTRUCTURE ONLY.

This module is a clean-room NumPy restatement of the reference algorithm
(liukefan821/adakv).  It is the checker the HIP path is compared against and
the CPU baseline timed by ``bench.py``; it is never imported by the product
package ``adakv_amd`` (which fails loudly without its HIP library).  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg use it.

Layout convention (same as the reference): ``[n_heads, seq_len, head_dim]``.

Every function cites the reference file:line whose semantics it restates.
Numerics follow the reference's NumPy 2 dtype rules exactly:

* block centroid = sequential fp32 sum over the block's real tokens, then a
  correctly rounded divide by the token count (``keys[:, s:e].mean(axis=1)``,
  estimator.py:45-47);
* scores are fp32 ``einsum`` (estimator.py:74);
* the entropy sum is fp32, the division by ``np.log(nb)`` (a float64 scalar)
  promotes everything after it to fp64, and ``np.round`` is half-to-even
  (budget.py:31-37, 83-86);
* selection ranks fp64 copies of the scores, sink/local forced via ``+inf``
  (selector.py:44-60).

Pinning (see tests/test_oracle_golden.py, tests/test_oracle_properties.py and
tests/test_oracle_evict.py): golden vectors written by the real reference in
this container (tests/golden/make_golden.py) pin scores, weights, budgets,
masks and outputs; closed forms / brute force pin the centroid, the selection
and the attention; the eviction baselines (key importance, pool, retention,
frozen tables and attention) are pinned by closed forms (column totals, the
last key's weight), a brute force, SciPy's maximum_filter1d, a sort, and the
reference's own CPU scenarios.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "expand_gqa", "dense_attention", "build_block_summaries", "block_scores",
    "budget_weights", "budget_bounds", "allocate_budget", "select_blocks",
    "sparse_attention", "plan_table", "ref_from_table", "centroid_after_append",
    "selection_near_ties", "budget_near_half", "budget_extra",
    "key_importance", "h2o_key_importance", "maxpool_same", "snapkv_key_importance",
    "retain_block_sums", "retain_blocks", "retain_near_ties", "frozen_decode_mask",
    "frozen_sparse_attention",
]


def _softmax_rows(x: np.ndarray) -> np.ndarray:
    # reference.py:23-26 (max-subtracted exp, normalised by the row sum)
    y = np.exp(x - x.max(axis=-1, keepdims=True))
    return y / y.sum(axis=-1, keepdims=True)


def expand_gqa(x: np.ndarray, n_q_heads: int) -> np.ndarray:
    """KV-head array -> query-head array by group repeat (reference.py:29-33)."""
    n_kv = x.shape[0]
    if n_q_heads % n_kv:
        raise AssertionError("n_q_heads must be a multiple of n_kv_heads")
    return np.repeat(x, n_q_heads // n_kv, axis=0)


def dense_attention(q: np.ndarray, K: np.ndarray, V: np.ndarray) -> np.ndarray:
    """Single-query softmax attention, q:[H,D] K,V:[H,S,D] (reference.py:36-41)."""
    logits = np.einsum("hd,hsd->hs", q, K) / np.sqrt(q.shape[-1])
    return np.einsum("hs,hsd->hd", _softmax_rows(logits), V)


def build_block_summaries(keys: np.ndarray, block_size: int, kind: str = "centroid") -> dict:
    """Per-block key summaries over real tokens only (estimator.py:27-48).

    ``centroid``: mean key of each block; the trailing partial block divides
    by its true token count.  ``minmax``: per-dim min / max (estimator.py:50-57).
    """
    H, S, D = keys.shape
    nb = -(-S // block_size)
    if kind == "centroid":
        out = np.empty((H, nb, D), dtype=np.float32)
        for b in range(nb):
            lo, hi = b * block_size, min(S, (b + 1) * block_size)
            # fp32 row-by-row accumulation then one divide: identical to
            # ndarray.mean over a non-contiguous axis (estimator.py:47).
            acc = keys[:, lo].astype(np.float32, copy=True)
            for t in range(lo + 1, hi):
                acc += keys[:, t]
            out[:, b] = acc / np.float32(hi - lo)
        return {"kind": "centroid", "n_blocks": nb, "n_real": S, "centroid": out}
    if kind == "minmax":
        kmin = np.empty((H, nb, D), dtype=np.float32)
        kmax = np.empty((H, nb, D), dtype=np.float32)
        for b in range(nb):
            blk = keys[:, b * block_size:min(S, (b + 1) * block_size)]
            kmin[:, b] = blk.min(axis=1)
            kmax[:, b] = blk.max(axis=1)
        return {"kind": "minmax", "n_blocks": nb, "n_real": S, "kmin": kmin, "kmax": kmax}
    raise ValueError(f"unknown estimator kind: {kind!r}")


def block_scores(q: np.ndarray, summ: dict) -> np.ndarray:
    """Block importance for the decode query (estimator.py:62-79).

    centroid: ``q . centroid`` (fp32 einsum, no 1/sqrt(D));
    minmax: Quest upper bound ``sum max(q,0)*kmax + min(q,0)*kmin``.
    """
    if summ["kind"] == "centroid":
        return np.einsum("hd,hbd->hb", q, summ["centroid"])
    qp = np.clip(q, 0.0, None)[:, None, :]
    qn = np.clip(q, None, 0.0)[:, None, :]
    return (qp * summ["kmax"] + qn * summ["kmin"]).sum(-1)


def budget_weights(scores: np.ndarray, policy: str = "adaptive", temperature: float = 1.0,
                   nucleus_p: float = 0.9) -> np.ndarray:
    """Per-head surplus weights (budget.py:28-42).

    adaptive: normalised softmax entropy + 1e-6 (fp32 sum, fp64 after the
    ``/ np.log(nb)``); adaptive_nucleus: #blocks whose cumulative sorted mass
    stays below ``nucleus_p``, plus one.
    """
    nb = scores.shape[1]
    z = scores / max(temperature, 1e-6)
    p = np.exp(z - z.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    if policy == "adaptive":
        h32 = -(p * np.log(np.clip(p, 1e-9, None))).sum(axis=-1)
        return h32 / np.log(max(nb, 2)) + 1e-6
    if policy == "adaptive_nucleus":
        srt = np.sort(p, axis=-1)[:, ::-1]
        return (np.cumsum(srt, axis=-1) < nucleus_p).sum(axis=-1).astype(np.float64) + 1.0
    raise ValueError(f"unknown budget policy: {policy!r}")


def budget_bounds(nb: int, avg_budget, k_min: int, k_max: int, n_sink_blocks: int,
                  n_local_blocks: int, c_min: int):
    """(lo, hi, target, floor_sel) as ``sparse_attention`` feeds them to the
    allocator and selector (reference.py:71-74, budget.py:72-77, selector.py:49-52)."""
    kmin_a, kmax_a = min(k_min, nb), min(k_max, nb)
    floor_arg = min(n_sink_blocks, nb) + min(n_local_blocks, nb) + c_min
    lo = min(max(int(floor_arg), int(kmin_a), 1), nb)
    hi = min(int(kmax_a), nb)
    target = float(np.clip(avg_budget, lo, hi))
    floor_sel = min(min(n_sink_blocks, nb) + min(n_local_blocks, nb) + c_min, nb)
    return lo, hi, target, floor_sel


def budget_extra(w: np.ndarray, lo: int, target: float) -> np.ndarray:
    """Unrounded per-head share above ``lo`` (budget.py:83-84), fp64."""
    H = w.shape[0]
    return max(target - lo, 0.0) * H * w / max(float(w.sum()), 1e-9)


def allocate_budget(scores: np.ndarray, avg_budget, k_min: int, k_max: int,
                    temperature: float = 1.0, policy: str = "adaptive",
                    nucleus_p: float = 0.9, floor: int | None = None) -> np.ndarray:
    """Mean-pinned per-head block budget (budget.py:45-86)."""
    H, nb = scores.shape
    if nb <= 1:
        return np.full((H,), min(max(k_min, 1), nb), dtype=np.int64)
    lo = min(max(int(k_min if floor is None else floor), int(k_min), 1), nb)
    hi = min(int(k_max), nb)
    target = float(np.clip(avg_budget, lo, hi))
    if policy == "fixed":
        return np.full((H,), int(round(target)), dtype=np.int64)
    w = budget_weights(scores, policy, temperature, nucleus_p)
    return np.clip(np.round(lo + budget_extra(w, lo, target)), lo, hi).astype(np.int64)


def select_blocks(scores: np.ndarray, k_per_head: np.ndarray, n_sink_blocks: int = 1,
                  n_local_blocks: int = 4, c_min: int = 1):
    """Forced sink/local + top-scoring fill to k_h -> (mask[H,nb], counts[H])
    (selector.py:18-60)."""
    H, nb = scores.shape
    sink, local = min(n_sink_blocks, nb), min(n_local_blocks, nb)
    ranked = scores.astype(np.float64, copy=True)
    if sink:
        ranked[:, :sink] = np.inf
    if local:
        ranked[:, nb - local:] = np.inf
    order = np.argsort(-ranked, axis=1)
    floor = min(sink + local + c_min, nb)
    mask = np.zeros((H, nb), dtype=bool)
    for h in range(H):
        take = min(max(int(k_per_head[h]), floor), nb)
        mask[h, order[h, :take]] = True
        mask[h, :sink] = True
        if local:
            mask[h, nb - local:] = True
    return mask, mask.sum(axis=1)


def sparse_attention(q, K, V, block_size=16, avg_budget=8, k_min=2, k_max=64,
                     estimator="centroid", n_sink_blocks=1, n_local_blocks=4, c_min=1,
                     budget_policy="adaptive", nucleus_p=0.9, return_mask=False,
                     return_all=False, temperature=1.0):
    """The AdaKV decode-step oracle (reference.py:44-84).

    q:[H,D], K,V:[H,S,D] already GQA-expanded.  Returns ``(out, counts)``
    (+ ``mask``), or with ``return_all`` a dict of every intermediate.
    ``temperature`` is fixed at 1.0 in the reference oracle; the runtime
    planner exposes it (attention.py:157,215), so it is a keyword here.
    """
    H, S, D = K.shape
    summ = build_block_summaries(K, block_size, estimator)
    scores = block_scores(q, summ)
    nb = summ["n_blocks"]
    k = allocate_budget(scores, avg_budget, min(k_min, nb), min(k_max, nb),
                        temperature=temperature, policy=budget_policy, nucleus_p=nucleus_p,
                        floor=min(n_sink_blocks, nb) + min(n_local_blocks, nb) + c_min)
    mask, counts = select_blocks(scores, k, n_sink_blocks, n_local_blocks, c_min)
    tok = np.repeat(mask, block_size, axis=1)[:, :S]
    logits = np.einsum("hd,hsd->hs", q, K) / np.sqrt(D)
    logits = np.where(tok, logits, -np.inf)
    out = np.einsum("hs,hsd->hd", _softmax_rows(logits), V)
    if return_all:
        return {"summ": summ, "scores": scores, "k": k, "mask": mask, "counts": counts,
                "out": out}
    if return_mask:
        return out, counts, mask
    return out, counts


def plan_table(scores: np.ndarray, k_per_head: np.ndarray, n_sink_blocks: int,
               n_local_blocks: int, c_min: int):
    """Selection as the runtime hands it to the kernel (attention.py:228-244):
    rows list the forced blocks first, then content blocks by descending score;
    only the first ``sel_lens[h]`` entries are valid.  Forced blocks are listed
    in ascending index order (the reference's +inf ties have no defined order)
    and equal content scores by ascending index."""
    H, nb = scores.shape
    sink, local = min(n_sink_blocks, nb), min(n_local_blocks, nb)
    forced = sorted(set(range(sink)) | set(range(nb - local, nb)))
    fset = set(forced)
    floor = min(sink + local + c_min, nb)
    content = np.array([b for b in range(nb) if b not in fset], dtype=np.int64)
    table = np.zeros((H, nb), dtype=np.int32)
    lens = np.zeros((H,), dtype=np.int32)
    for h in range(H):
        s64 = scores[h, content].astype(np.float64)
        order = content[np.lexsort((content, -s64))]
        row = np.concatenate([np.array(forced, dtype=np.int64), order])
        table[h] = row
        lens[h] = min(max(int(k_per_head[h]), floor), nb)
    return table, lens


def ref_from_table(q, k, v, block_table, sel_lens, block_size, group, sm_scale=None):
    """fp32 attention over exactly the listed blocks, duplicates counted once
    (tests/test_kernel_parity.py:25-43).  q:[Hq,D], k,v:[Hkv,S,D]."""
    Hq, D = q.shape
    S = k.shape[1]
    scale = (1.0 / np.sqrt(D)) if sm_scale is None else sm_scale
    out = np.zeros((Hq, D), dtype=np.float32)
    for h in range(Hq):
        g = h // group
        toks = set()
        for j in range(int(sel_lens[h])):
            b = int(block_table[h, j])
            toks.update(range(b * block_size, min((b + 1) * block_size, S)))
        idx = np.array(sorted(t for t in toks if 0 <= t < S), dtype=np.int64)
        if idx.size == 0:
            out[h] = np.nan
            continue
        s = (k[g, idx].astype(np.float64) @ q[h].astype(np.float64)) * scale
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ v[g, idx].astype(np.float64)
    return out


def centroid_after_append(centroid: np.ndarray, n_before: int, k_t: np.ndarray,
                          block_size: int) -> np.ndarray:
    """Running-mean centroid update for one appended token (runtime.py:43-60).

    k_t:[H,D].  A token that opens a new block appends it as that block's
    centroid; otherwise ``mu + (x - mu) / (count_before + 1)``.
    """
    b = n_before // block_size
    cnt = n_before - b * block_size
    if b >= centroid.shape[1]:
        return np.concatenate([centroid, k_t[:, None, :].astype(centroid.dtype)], axis=1)
    out = centroid.copy()
    mu = out[:, b]
    out[:, b] = mu + (k_t - mu) / (cnt + 1)
    return out


# --------------------------------------------------------------------------
# Near-tie classification.  The oracle's einsum accumulation order is NumPy's
# SIMD detail and cannot be reproduced by any other summation; bit-exact
# selection parity is therefore asserted on every head except those whose
# decision sits within rounding distance of a tie.
# --------------------------------------------------------------------------
def selection_near_ties(scores: np.ndarray, k_per_head: np.ndarray, n_sink_blocks: int,
                        n_local_blocks: int, c_min: int, rel_tol: float = 1e-5,
                        abs_scale: np.ndarray | None = None) -> np.ndarray:
    """Per-head flag: the k-th / (k+1)-th content scores are within
    ``rel_tol * scale`` of each other (scale = max|score| of the head, or
    ``abs_scale[h]`` when given)."""
    H, nb = scores.shape
    sink, local = min(n_sink_blocks, nb), min(n_local_blocks, nb)
    forced = set(range(sink)) | set(range(nb - local, nb))
    content = np.array([b for b in range(nb) if b not in forced], dtype=np.int64)
    floor = min(sink + local + c_min, nb)
    flags = np.zeros((H,), dtype=bool)
    for h in range(H):
        take = min(max(int(k_per_head[h]), floor), nb) - len(forced)
        if content.size == 0 or take <= 0 or take >= content.size:
            continue
        s = np.sort(scores[h, content].astype(np.float64))[::-1]
        scale = float(np.abs(scores[h]).max()) if abs_scale is None else float(abs_scale[h])
        flags[h] = (s[take - 1] - s[take]) <= rel_tol * max(scale, 1e-30)
    return flags


def budget_near_half(w: np.ndarray, lo: int, target: float, margin: float = 1e-3) -> np.ndarray:
    """Per-head flag: ``lo + extra`` lies within ``margin`` of a .5 rounding
    boundary (budget.py:85), where a last-ulp change of the weights flips k."""
    x = lo + budget_extra(np.asarray(w, dtype=np.float64), lo, target)
    return np.abs((x - np.floor(x)) - 0.5) <= margin


# --------------------------------------------------------------------------
# Eviction baselines (H2O, SnapKV): a retained block set frozen at prefill
# from the prompt's own attention (adakv/baselines.py, adakv/baselines_rt.py).
# Q, K are [H, S, D] expanded to query heads, as in the reference.
# --------------------------------------------------------------------------
def key_importance(Q: np.ndarray, K: np.ndarray, first_query: int = 0) -> np.ndarray:
    """Attention each key receives, summed over the causal queries at
    positions [first_query, S): fp64 logits q_i . k_j / sqrt(D) for j <= i,
    row softmax over keys, column sums, fp32 result [H, S].

    first_query = 0 is H2O's accumulated attention (baselines.py:63-79);
    first_query = S - min(obs_window, S) is SnapKV's window before its pool
    (baselines.py:101-114).  Rows are processed in slices so that only
    [H, rows, S] is live at once."""
    H, S, D = K.shape
    if Q.shape != (H, S, D):
        raise AssertionError("Q and K must share [H, S, D]")
    first_query = int(min(max(first_query, 0), S))
    Kd = K.astype(np.float64)
    inv = 1.0 / np.sqrt(D)
    imp = np.zeros((H, S), dtype=np.float64)
    keys = np.arange(S)
    step = 256
    for i0 in range(first_query, S, step):
        i1 = min(i0 + step, S)
        logits = np.einsum("hid,hjd->hij", Q[:, i0:i1].astype(np.float64), Kd) * inv
        visible = keys[None, :] <= np.arange(i0, i1)[:, None]           # key j <= query i
        logits = np.where(visible[None], logits, -np.inf)
        imp += _softmax_rows(logits).sum(axis=1)
    return imp.astype(np.float32)


def h2o_key_importance(Q: np.ndarray, K: np.ndarray) -> np.ndarray:
    """H2O heavy-hitter signal: every prompt query (baselines.py:63-79)."""
    return key_importance(Q, K, 0)


def maxpool_same(x: np.ndarray, kernel: int) -> np.ndarray:
    """Same-length max over the window [t - kernel//2, t + kernel//2] of the
    last axis, clipped to the array (edge padding, baselines.py:82-92; for a
    max, equal to torch's -inf padding, baselines_rt.py:79-80)."""
    if kernel <= 1:
        return x
    r = kernel // 2
    S = x.shape[-1]
    out = np.empty_like(x)
    for t in range(S):
        out[..., t] = x[..., max(0, t - r):min(S, t + r + 1)].max(axis=-1)
    return out


def snapkv_key_importance(Q: np.ndarray, K: np.ndarray, obs_window: int = 32,
                          pool_kernel: int = 7) -> np.ndarray:
    """SnapKV: attention from the last obs_window queries, max-pooled over
    key positions (baselines.py:95-115)."""
    S = K.shape[1]
    w = int(min(obs_window, S))
    return maxpool_same(key_importance(Q, K, S - w), pool_kernel).astype(np.float32)


def retain_block_sums(importance: np.ndarray, block_size: int, n_real: int) -> np.ndarray:
    """fp64 sum of each block's importance over its real tokens (baselines.py:139-143)."""
    H = importance.shape[0]
    nb = -(-n_real // block_size)
    blk = np.zeros((H, nb), dtype=np.float64)
    for b in range(nb):
        s, e = b * block_size, min((b + 1) * block_size, n_real)
        blk[:, b] = importance[:, s:e].astype(np.float64).sum(axis=1)
    return blk


def retain_blocks(importance: np.ndarray, block_size: int, n_real: int, budget: int,
                  n_sink_blocks: int = 1, n_local_blocks: int = 4, c_min: int = 1) -> np.ndarray:
    """Frozen retained mask [H, nb]: k = min(max(budget, floor), nb) blocks
    per head -- the sink and local blocks, then the content blocks of largest
    block sum (baselines.py:120-160).  Equal sums are taken in ascending block
    order (a stable descending sort); the reference's unstable argsort leaves
    that order unspecified, so tests exclude near-ties."""
    blk = retain_block_sums(importance, block_size, n_real)
    H, nb = blk.shape
    sink, local = min(n_sink_blocks, nb), min(n_local_blocks, nb)
    biased = blk.copy()
    biased[:, :sink] = np.inf
    if local:
        biased[:, nb - local:] = np.inf
    floor = min(sink + local + c_min, nb)
    k = min(max(int(budget), floor), nb)
    mask = np.zeros((H, nb), dtype=bool)
    for h in range(H):
        mask[h, np.argsort(-biased[h], kind="stable")[:k]] = True
        mask[h, :sink] = True
        if local:
            mask[h, nb - local:] = True
    return mask


def retain_near_ties(importance: np.ndarray, block_size: int, n_real: int, budget: int,
                     n_sink_blocks: int, n_local_blocks: int, c_min: int,
                     rel_tol: float = 1e-5) -> np.ndarray:
    """Per-head flag: the last retained and first evicted content block sums
    are within rel_tol * (largest block sum of the head)."""
    blk = retain_block_sums(importance, block_size, n_real)
    H, nb = blk.shape
    sink, local = min(n_sink_blocks, nb), min(n_local_blocks, nb)
    content = np.arange(sink, max(nb - local, sink))
    k = min(max(int(budget), min(sink + local + c_min, nb)), nb)
    take = k - (sink + len(set(range(nb - local, nb)) - set(range(sink))))
    flags = np.zeros((H,), dtype=bool)
    if content.size == 0 or take <= 0 or take >= content.size:
        return flags
    for h in range(H):
        s = np.sort(blk[h, content])[::-1]
        flags[h] = (s[take - 1] - s[take]) <= rel_tol * max(float(blk[h].max()), 1e-30)
    return flags


def frozen_decode_mask(fmask: np.ndarray, nb_now: int, n_sink_blocks: int,
                       n_local_blocks: int) -> np.ndarray:
    """Decode-time retained set [H, nb_now]: the frozen prefill set plus the
    sink and the local window of the current blocks (baselines_rt.py:182-205)."""
    H, nbp = fmask.shape
    if nb_now < nbp:
        raise AssertionError("decode block count must not shrink below prefill")
    sink, local = min(n_sink_blocks, nb_now), min(n_local_blocks, nb_now)
    m = np.zeros((H, nb_now), dtype=bool)
    m[:, :nbp] = fmask
    m[:, :sink] = True
    if local:
        m[:, nb_now - local:] = True
    return m


def frozen_sparse_attention(q: np.ndarray, K: np.ndarray, V: np.ndarray, retained_mask: np.ndarray,
                            block_size: int):
    """One decode step over the retained blocks only (baselines.py:197-212):
    (out [H, D], counts [H])."""
    H, S, D = K.shape
    tok = np.repeat(retained_mask, block_size, axis=1)[:, :S]
    logits = np.einsum("hd,hsd->hs", q, K) / np.sqrt(D)
    out = np.einsum("hs,hsd->hd", _softmax_rows(np.where(tok, logits, -np.inf)), V)
    return out, retained_mask.sum(axis=1)
