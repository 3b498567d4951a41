"""Helpers shared by the GPU parity tests (selection comparison with near-tie
exclusion, tensor plumbing)."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle import adakv_oracle as O

torch = pytest.importorskip("torch")

DEV = "cuda"

# bf16 output tolerance (fp32 accumulation), as stated by the north star.
BF16_ATOL = 2e-2
REL_L2 = 2e-2


def say(msg: str) -> None:
    """Name the case before each GPU step (flushed, so a fault still shows it)."""
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from adakv_amd import _capi
    _capi.load()  # raises if the library is missing: no silent fallback


def to_np(t) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def gpu_sets(table: np.ndarray, lens: np.ndarray):
    return [set(int(x) for x in table[h, : int(lens[h])]) for h in range(table.shape[0])]


def compare_selection(scores: np.ndarray, table: np.ndarray, lens: np.ndarray, *, k_oracle,
                      w_oracle, lo, target, sink, local, cmin, policy, max_excluded=0.25,
                      tie_tol=1e-5, exclude=None, half_margin=1e-3):
    """Check a GPU selection against the oracle for one sequence.

    scores: oracle fp32 scores [H, nb]; table/lens: GPU output for the same heads.
    * sel_lens must equal the oracle's (post-floor) count on every head whose
      unrounded budget is not within 1e-3 of a .5 boundary;
    * the selected set must equal the oracle's selection at the GPU's own count
      on every head without a score near-tie at that boundary;
    * forced blocks come first in ascending order and content entries are in
      non-increasing oracle score order (up to near-ties).
    Returns the number of excluded heads.
    """
    H, nb = scores.shape
    floor = min(min(sink, nb) + min(local, nb) + cmin, nb)
    k_exp = np.minimum(np.maximum(k_oracle, floor), nb)
    if policy in ("adaptive", "adaptive_nucleus") and nb > 1:
        near_half = O.budget_near_half(w_oracle, lo, target, margin=half_margin)
    else:
        near_half = np.zeros(H, bool)
    if exclude is not None:
        near_half = near_half | exclude
    bad = [(h, int(lens[h]), int(k_exp[h])) for h in range(H)
           if not near_half[h] and int(lens[h]) != int(k_exp[h])]
    assert not bad, f"sel_lens differ from the oracle on heads {bad[:8]}"
    ties = O.selection_near_ties(scores, lens, sink, local, cmin, rel_tol=tie_tol)
    mask, _ = O.select_blocks(scores, lens.astype(np.int64), sink, local, cmin)
    sets = gpu_sets(table, lens)
    sink_n, local_n = min(sink, nb), min(local, nb)
    forced = sorted(set(range(sink_n)) | set(range(nb - local_n, nb)))
    mism = []
    for h in range(H):
        if ties[h]:
            continue
        if sets[h] != set(np.flatnonzero(mask[h]).tolist()):
            mism.append(h)
            continue
        row = [int(x) for x in table[h, : int(lens[h])]]
        assert row[: len(forced)] == forced[: len(row)], f"head {h}: forced prefix {row[:8]}"
        cont = np.array(row[len(forced):], dtype=np.int64)
        if cont.size > 1:
            s = scores[h, cont].astype(np.float64)
            tol = tie_tol * max(float(np.abs(scores[h]).max()), 1e-30)
            assert np.all(np.diff(s) <= tol), f"head {h}: content not in descending score order"
    assert not mism, f"selection differs from the oracle on heads {mism[:8]}"
    excluded = int(np.sum(near_half | ties))
    assert excluded <= max_excluded * H, f"{excluded}/{H} heads excluded as near-ties"
    return excluded


def nucleus_ambiguous(scores: np.ndarray, temperature: float = 1.0, nucleus_p: float = 0.9,
                      tol: float = 1e-6, per_term: float = 6e-8) -> np.ndarray:
    """Per-head flag: the nucleus count (adakv/budget.py:38-41) depends on the
    rounding of the cumulative sums -- the exact (fp64) sum of the top K* or
    K* - 1 probabilities lies within tol + K* * per_term of P (the worst-case
    error of NumPy's fp32 running sum over K* terms, half an ulp of 1 each,
    plus the last-ulp differences of p between NumPy and the GPU), where
    NumPy's sum and the GPU's exact integer masses may land on either side."""
    w = O.budget_weights(scores, "adaptive_nucleus", temperature, nucleus_p)
    z = scores / max(temperature, 1e-6)
    p = np.exp(z - z.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    c = np.cumsum(np.sort(p.astype(np.float64), axis=-1)[:, ::-1], axis=-1)
    P = float(np.float32(nucleus_p))
    nb = scores.shape[1]
    out = np.zeros(scores.shape[0], bool)
    for h in range(scores.shape[0]):
        k = int(w[h])                       # K*: the crossing is the k-th largest
        for j in (k - 2, k - 1):
            if 0 <= j < nb and abs(c[h, j] - P) <= tol + k * per_term:
                out[h] = True
    return out


def nucleus_exclusions(scores: np.ndarray, lo: int, target: float, temperature: float = 1.0,
                       nucleus_p: float = 0.9):
    """(heads to exclude, near-half margin) for comparing nucleus budgets: the
    knife-edge heads themselves, and for every other head a rounding margin
    wide enough for their weights moving by one (which moves the sum of weights
    every share is divided by)."""
    amb = nucleus_ambiguous(scores, temperature, nucleus_p)
    w = O.budget_weights(scores, "adaptive_nucleus", temperature, nucleus_p)
    extra = O.budget_extra(w, lo, target)
    shift = 2.0 * float(amb.sum()) * float(extra.max(initial=0.0)) / max(float(w.sum()), 1e-9)
    return amb, max(1e-3, shift + 1e-4)


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-12))
