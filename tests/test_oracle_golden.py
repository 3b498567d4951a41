"""The CPU oracle against the golden vectors written by the real reference.

The fixtures (tests/golden/*.npz) were produced by tests/golden/make_golden.py,
which imports the reference's own NumPy modules.  Passing here pins every
oracle function the path uses: centroid (checksum), fp32 scores, fp64 weights,
round-half-even budgets, masks, counts and the attention output.  The mutation
tests below plant plausible mistakes in copies of the oracle and require the
same checks to catch each one.
"""
from __future__ import annotations

import os
import types

import numpy as np
import pytest

import cases
import golden_check
from oracle import adakv_oracle as O

CASE_NAMES = sorted(cases.CASES)


@pytest.mark.parametrize("name", CASE_NAMES)
def test_oracle_matches_reference_golden(name):
    assert golden_check.check_case(O, name) == []


@pytest.mark.parametrize("name", ["cfg1_seed0", "gqa6_kmax256"])
def test_plan_table_matches_reference_planner(name):
    """Runtime planner format (attention.py:228-244): same selected set per head,
    forced blocks first, content in the same descending-score order."""
    p = cases.params(name)
    with np.load(os.path.join(golden_check.GOLDEN, f"plan_{name}.npz")) as z:
        bt, sl = z["block_table"], z["sel_lens"]
    g = golden_check.load(name)
    table, lens = O.plan_table(g["scores"], g["k"], p["sink"], p["local"], p["cmin"])
    assert np.array_equal(lens, sl)
    nb = g["scores"].shape[1]
    nforced = len(set(range(min(p["sink"], nb))) | set(range(nb - min(p["local"], nb), nb)))
    for h in range(table.shape[0]):
        n = int(lens[h])
        assert set(table[h, :n].tolist()) == set(bt[h, :n].tolist())
        assert set(table[h, :nforced].tolist()) == set(bt[h, :nforced].tolist())
        assert table[h, nforced:n].tolist() == bt[h, nforced:n].tolist()


# ---- mutation tests: each planted mistake must be caught ---------------------

def _mutant(**overrides):
    m = types.SimpleNamespace(**{k: getattr(O, k) for k in O.__all__})
    for k, v in overrides.items():
        setattr(m, k, v)
    # sparse_attention must call the mutated pieces: rebuild it over the namespace
    def sparse_attention(q, K, V, block_size=16, avg_budget=8, k_min=2, k_max=64,
                         estimator="centroid", n_sink_blocks=1, n_local_blocks=4, c_min=1,
                         budget_policy="adaptive", nucleus_p=0.9, return_mask=False,
                         return_all=False, temperature=1.0):
        H, S, D = K.shape
        summ = m.build_block_summaries(K, block_size, estimator)
        scores = m.block_scores(q, summ)
        nb = summ["n_blocks"]
        k = m.allocate_budget(scores, avg_budget, min(k_min, nb), min(k_max, nb),
                              temperature=temperature, policy=budget_policy,
                              nucleus_p=nucleus_p,
                              floor=min(n_sink_blocks, nb) + min(n_local_blocks, nb) + c_min)
        mask, counts = m.select_blocks(scores, k, n_sink_blocks, n_local_blocks, c_min)
        tok = np.repeat(mask, block_size, axis=1)[:, :S]
        logits = np.where(tok, np.einsum("hd,hsd->hs", q, K) / m.attn_scale(D), -np.inf)
        e = np.exp(logits - logits.max(axis=-1, keepdims=True))
        out = np.einsum("hs,hsd->hd", e / e.sum(axis=-1, keepdims=True), V)
        return {"summ": summ, "scores": scores, "k": k, "mask": mask, "counts": counts,
                "out": out}
    m.sparse_attention = sparse_attention
    if not hasattr(m, "attn_scale"):
        m.attn_scale = np.sqrt
    return m


def _centroid_divide_by_bs(keys, bs, kind="centroid"):
    H, S, D = keys.shape
    nb = -(-S // bs)
    pad = np.zeros((H, nb * bs - S, D), np.float32)
    c = np.concatenate([keys, pad], 1).reshape(H, nb, bs, D).sum(2) / np.float32(bs)
    return {"kind": "centroid", "n_blocks": nb, "n_real": S, "centroid": c.astype(np.float32)}


def _scores_scaled(q, summ):
    return O.block_scores(q, summ) / np.float32(np.sqrt(q.shape[-1]))


def _weights_no_norm(scores, policy="adaptive", temperature=1.0, nucleus_p=0.9):
    if policy != "adaptive":
        return O.budget_weights(scores, policy, temperature, nucleus_p)
    return O.budget_weights(scores, policy, temperature, nucleus_p) * np.log(scores.shape[1])


def _alloc_floor(scores, avg_budget, k_min, k_max, temperature=1.0, policy="adaptive",
                 nucleus_p=0.9, floor=None):
    H, nb = scores.shape
    if nb <= 1 or policy == "fixed":
        return O.allocate_budget(scores, avg_budget, k_min, k_max, temperature, policy,
                                 nucleus_p, floor)
    lo = min(max(int(floor), int(k_min), 1), nb)
    hi = min(int(k_max), nb)
    target = float(np.clip(avg_budget, lo, hi))
    w = O.budget_weights(scores, policy, temperature, nucleus_p)
    return np.clip(np.floor(lo + O.budget_extra(w, lo, target)), lo, hi).astype(np.int64)


def _minmax_bounds_swapped(q, summ):
    if summ["kind"] != "minmax":
        return O.block_scores(q, summ)
    return O.block_scores(q, dict(summ, kmax=summ["kmin"], kmin=summ["kmax"]))


def _minmax_from_padded_blocks(keys, bs, kind="centroid"):
    if kind != "minmax":
        return O.build_block_summaries(keys, bs, kind)
    H, S, D = keys.shape
    nb = -(-S // bs)
    kp = np.concatenate([keys, np.zeros((H, nb * bs - S, D), np.float32)], 1).reshape(H, nb, bs, D)
    return {"kind": "minmax", "n_blocks": nb, "n_real": S, "kmin": kp.min(2), "kmax": kp.max(2)}


def _select_no_local(scores, k, n_sink_blocks=1, n_local_blocks=4, c_min=1):
    return O.select_blocks(scores, k, n_sink_blocks, 0, c_min + n_local_blocks)


def _select_ascending(scores, k, n_sink_blocks=1, n_local_blocks=4, c_min=1):
    return O.select_blocks(-scores, k, n_sink_blocks, n_local_blocks, c_min)


MUTANTS = {
    "centroid_divides_partial_block_by_block_size": dict(build_block_summaries=_centroid_divide_by_bs),
    "scores_scaled_by_inv_sqrt_d": dict(block_scores=_scores_scaled),
    "entropy_not_normalised": dict(budget_weights=_weights_no_norm),
    "budget_floor_instead_of_round": dict(allocate_budget=_alloc_floor),
    "local_window_not_forced": dict(select_blocks=_select_no_local),
    "selection_sign_flipped": dict(select_blocks=_select_ascending),
    "attention_scale_missing": dict(attn_scale=lambda d: 1.0),
    "minmax_bounds_swapped": dict(block_scores=_minmax_bounds_swapped),
}



@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_planted_mistake_is_caught(mutant):
    m = _mutant(**MUTANTS[mutant])
    caught = []
    for name in ("partial_tail", "cfg1_seed0", "temp_sink_local", "peaked_mixed", "minmax_fixed"):
        caught += golden_check.check_case(m, name)
    assert caught, f"mutant {mutant} passed the golden checks"


def test_minmax_padding_mistake_is_caught_by_a_closed_form():
    """A partial last block padded with zeros before min / max: the bounds of
    one-token blocks must equal the token itself."""
    rng = np.random.default_rng(3)
    K = (rng.standard_normal((2, 33, 8)).astype(np.float32) + np.float32(5.0))   # all positive
    for build, ok in ((O.build_block_summaries, True), (_minmax_from_padded_blocks, False)):
        s = build(K, 16, "minmax")
        exact = np.array_equal(s["kmin"][:, 2], K[:, 32]) and np.array_equal(s["kmax"][:, 2], K[:, 32])
        assert exact == ok
