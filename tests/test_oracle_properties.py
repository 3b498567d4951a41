"""Oracle checks fixed by mathematics rather than by the golden vectors.

Re-expresses the reference's own CPU tests (tests/test_reference.py,
tests/test_factorial_selection.py, tests/test_runtime_cpu.py) against the
clean-room oracle, plus closed forms and brute force on tiny inputs.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest

from oracle import adakv_oracle as O


def _case(H=4, S=512, D=64, planted_block=7, bs=16, seed=0):
    # tests/test_reference.py:24-32 pattern
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((H, D)).astype(np.float32)
    K = rng.standard_normal((H, S, D)).astype(np.float32) * np.float32(0.1)
    V = rng.standard_normal((H, S, D)).astype(np.float32)
    K[:, planted_block * bs:(planted_block + 1) * bs] = q[:, None, :] * np.float32(3.0)
    return q, K, V


def test_gqa_expand_groups():
    K = np.random.default_rng(1).standard_normal((2, 64, 8)).astype(np.float32)
    E = O.expand_gqa(K, 8)
    assert E.shape == (8, 64, 8)
    assert np.array_equal(E[0], E[3]) and np.array_equal(E[4], E[7])
    assert not np.array_equal(E[3], E[4])
    with pytest.raises(AssertionError):
        O.expand_gqa(K, 7)


def test_forced_sink_and_local_always_selected():
    q, K, V = _case()
    _, _, mask = O.sparse_attention(q, K, V, avg_budget=6, n_sink_blocks=2, n_local_blocks=3,
                                    return_mask=True)
    assert mask[:, :2].all() and mask[:, -3:].all()


def test_planted_block_recovered_by_every_head():
    q, K, V = _case(planted_block=7)
    _, _, mask = O.sparse_attention(q, K, V, avg_budget=6, n_sink_blocks=1, n_local_blocks=2,
                                    return_mask=True)
    assert mask[:, 7].all()


def test_full_budget_equals_dense_and_small_budget_is_close():
    q, K, V = _case()
    nb = 512 // 16
    dense = O.dense_attention(q, K, V)
    full, _ = O.sparse_attention(q, K, V, avg_budget=nb, k_min=nb, k_max=nb)
    assert np.allclose(dense, full, atol=1e-4)
    small, counts = O.sparse_attention(q, K, V, avg_budget=6)
    assert np.linalg.norm(dense - small) / np.linalg.norm(dense) < 0.05
    assert counts.max() <= nb


def test_flat_heads_get_more_budget_than_peaked():
    rng = np.random.default_rng(3)
    s = (rng.standard_normal((8, 64)) * 0.01).astype(np.float32)
    s[:4, 0] += 30.0
    k = O.allocate_budget(s, 8, 2, 48)
    assert k[:4].mean() < k[4:].mean() and k.min() >= 2 and k.max() <= 48


def test_centroid_closed_form_and_partial_block():
    rng = np.random.default_rng(5)
    S, bs = 37, 16                       # blocks of 16, 16, 5 tokens
    K = rng.integers(-8, 8, size=(3, S, 4)).astype(np.float32)   # exact in fp32
    c = O.build_block_summaries(K, bs)["centroid"]
    for b, (lo, hi) in enumerate([(0, 16), (16, 32), (32, 37)]):
        exact = K[:, lo:hi].astype(np.float64).sum(1) / (hi - lo)
        assert np.array_equal(c[:, b], exact.astype(np.float32))


def test_centroid_is_sequential_fp32_sum_then_divide():
    """ndarray.mean over the token axis == sequential fp32 accumulation / count."""
    rng = np.random.default_rng(6)
    K = rng.standard_normal((2, 48, 16)).astype(np.float32) * np.float32(1e3)
    c = O.build_block_summaries(K, 16)["centroid"]
    for b in range(3):
        acc = np.zeros((2, 16), np.float32)
        for t in range(16):
            acc = (acc + K[:, b * 16 + t]).astype(np.float32)
        assert np.array_equal(c[:, b], acc / np.float32(16))
        assert np.array_equal(c[:, b], K[:, b * 16:(b + 1) * 16].mean(axis=1))


def test_scores_match_fp64_brute_force():
    rng = np.random.default_rng(7)
    q = rng.standard_normal((4, 128)).astype(np.float32)
    c = rng.standard_normal((4, 64, 128)).astype(np.float32)
    s = O.block_scores(q, {"kind": "centroid", "centroid": c})
    ref = np.array([[float(np.dot(q[h].astype(np.float64), c[h, b].astype(np.float64)))
                     for b in range(64)] for h in range(4)])
    assert s.dtype == np.float32
    assert np.abs(s - ref).max() <= 1e-5 * np.abs(ref).max()


def test_minmax_bound_dominates_every_key_of_its_block():
    """Quest's bound (estimator.py:76-79) is >= q . k for every real key of the
    block, with equality for one-token blocks and for blocks whose keys are
    all equal; the bounds are the per-dimension extremes over real tokens."""
    rng = np.random.default_rng(11)
    H, S, D, bs = 3, 16 * 9 + 1, 32, 16          # last block: one token
    q = rng.standard_normal((H, D)).astype(np.float32)
    K = rng.standard_normal((H, S, D)).astype(np.float32)
    K[:, 16:32] = K[:, 16:17]                     # block 1: every key equal
    summ = O.build_block_summaries(K, bs, "minmax")
    nb = summ["n_blocks"]
    assert nb == 10
    for b in range(nb):
        blk = K[:, b * bs:min(S, (b + 1) * bs)]
        assert np.array_equal(summ["kmax"][:, b], blk.max(axis=1))
        assert np.array_equal(summ["kmin"][:, b], blk.min(axis=1))
    s = O.block_scores(q, summ).astype(np.float64)
    q64, K64 = q.astype(np.float64), K.astype(np.float64)
    for b in range(nb):
        dots = np.einsum("hd,hsd->hs", q64, K64[:, b * bs:min(S, (b + 1) * bs)])
        assert np.all(s[:, b] >= dots.max(axis=1) - 1e-4)
        if b in (1, nb - 1):
            assert np.allclose(s[:, b], dots[:, 0], rtol=0, atol=1e-4)
    # closed form on one dimension: q > 0 picks the max, q < 0 the min
    one = O.block_scores(np.array([[2.0, -3.0]], np.float32),
                         {"kind": "minmax", "kmax": np.array([[[1.0, 4.0]]], np.float32),
                          "kmin": np.array([[[-1.0, -2.0]]], np.float32)})
    assert one[0, 0] == np.float32(2.0 * 1.0 + -3.0 * -2.0)


def test_entropy_weight_closed_forms():
    flat = np.zeros((1, 256), np.float32)
    w = O.budget_weights(flat)
    assert w.dtype == np.float64 and abs(w[0] - (1.0 + 1e-6)) < 1e-6
    onehot = np.full((1, 256), -1e4, np.float32)
    onehot[0, 3] = 0.0
    assert abs(O.budget_weights(onehot)[0] - 1e-6) < 1e-9
    two = np.full((1, 256), -1e4, np.float32)
    two[0, :2] = 0.0                     # two equal blocks: H = log 2, normalised by log 256
    assert abs(O.budget_weights(two)[0] - (np.log(2) / np.log(256) + 1e-6)) < 1e-6


def test_budget_invariants_and_mean_pinning():
    rng = np.random.default_rng(8)
    for trial in range(20):
        H, nb = 32, int(rng.integers(8, 300))
        s = (rng.standard_normal((H, nb)) * rng.uniform(0.1, 5)).astype(np.float32)
        avg = int(rng.integers(1, 40))
        lo, hi, target, _ = O.budget_bounds(nb, avg, 2, 64, 1, 4, 1)
        k = O.allocate_budget(s, avg, min(2, nb), min(64, nb), floor=min(1, nb) + min(4, nb) + 1)
        assert k.min() >= min(lo, hi) and k.max() <= hi
        if lo <= hi and (k > lo).all() and (k < hi).all():
            # round() moves each head by at most 0.5 from its exact share
            assert abs(k.sum() - target * H) <= H / 2 + 1e-9
        kf = O.allocate_budget(s, avg, min(2, nb), min(64, nb), policy="fixed",
                               floor=min(1, nb) + min(4, nb) + 1)
        assert (kf == int(round(target))).all()


def test_fixed_budget_rounds_half_to_even():
    s = np.zeros((4, 64), np.float32)
    assert (O.allocate_budget(s, 8.5, 2, 64, policy="fixed", floor=6) == 8).all()
    assert (O.allocate_budget(s, 9.5, 2, 64, policy="fixed", floor=6) == 10).all()


def test_single_block_special_case():
    s = np.zeros((3, 1), np.float32)
    assert (O.allocate_budget(s, 8, 2, 64, floor=6) == 1).all()


@pytest.mark.parametrize("seed", range(12))
def test_selection_is_the_best_subset_by_brute_force(seed):
    rng = np.random.default_rng(seed)
    nb = int(rng.integers(3, 11))
    sink, local, cmin = int(rng.integers(0, 3)), int(rng.integers(0, 3)), 1
    s = rng.standard_normal((2, nb)).astype(np.float32)
    k = rng.integers(1, nb + 2, size=2)
    mask, counts = O.select_blocks(s, k, sink, local, cmin)
    forced = set(range(min(sink, nb))) | set(range(nb - min(local, nb), nb))
    content = [b for b in range(nb) if b not in forced]
    floor = min(min(sink, nb) + min(local, nb) + cmin, nb)
    for h in range(2):
        take = min(max(int(k[h]), floor), nb) - len(forced)
        best = max(itertools.combinations(content, take), key=lambda c: sum(s[h, list(c)]))
        assert set(np.flatnonzero(mask[h])) == forced | set(best)
        assert counts[h] == len(forced) + take


def test_no_content_starvation():
    # tests/test_factorial_selection.py:52-61: every head keeps >= c_min content blocks
    rng = np.random.default_rng(9)
    q = rng.standard_normal((12, 64)).astype(np.float32)
    K = O.expand_gqa(rng.standard_normal((2, 320, 64)).astype(np.float32), 12)
    for pol in ("fixed", "adaptive", "adaptive_nucleus"):
        for ab in (4, 6, 8):
            _, counts = O.sparse_attention(q, K, K, avg_budget=ab, k_max=256, n_sink_blocks=1,
                                           n_local_blocks=2, c_min=1, budget_policy=pol)
            assert (counts - 3).min() >= 1


def test_adaptive_mean_near_target():
    # tests/test_factorial_selection.py:71-76
    rng = np.random.default_rng(10)
    q = rng.standard_normal((12, 64)).astype(np.float32)
    K = O.expand_gqa(rng.standard_normal((2, 320, 64)).astype(np.float32), 12)
    for pol in ("adaptive", "adaptive_nucleus"):
        _, counts = O.sparse_attention(q, K, K, avg_budget=8, k_max=256, n_sink_blocks=1,
                                       n_local_blocks=2, c_min=1, budget_policy=pol)
        assert 4 <= counts.mean() <= 10


def test_ref_from_table_all_blocks_equals_dense():
    rng = np.random.default_rng(11)
    Hkv, G, S, D, bs = 2, 3, 100, 32, 16
    q = rng.standard_normal((Hkv * G, D)).astype(np.float32)
    k = rng.standard_normal((Hkv, S, D)).astype(np.float32)
    v = rng.standard_normal((Hkv, S, D)).astype(np.float32)
    nb = -(-S // bs)
    table = np.tile(np.arange(nb, dtype=np.int32)[::-1], (Hkv * G, 2))   # every block twice
    lens = np.full((Hkv * G,), 2 * nb, np.int32)
    out = O.ref_from_table(q, k, v, table, lens, bs, G)
    dense = O.dense_attention(q, O.expand_gqa(k, Hkv * G), O.expand_gqa(v, Hkv * G))
    assert np.allclose(out, dense, atol=1e-5)


def test_incremental_centroid_matches_recompute():
    # tests/test_runtime_cpu.py:34-44 (running mean vs recompute, < 1e-4)
    rng = np.random.default_rng(12)
    Hkv, S0, D, bs = 4, 100, 32, 16
    K = rng.standard_normal((Hkv, S0, D)).astype(np.float32)
    c = O.build_block_summaries(K, bs)["centroid"]
    for _ in range(50):
        kt = rng.standard_normal((Hkv, D)).astype(np.float32)
        c = O.centroid_after_append(c, K.shape[1], kt, bs)
        K = np.concatenate([K, kt[:, None]], axis=1)
    ref = O.build_block_summaries(K, bs)["centroid"]
    assert c.shape == ref.shape and np.abs(c - ref).max() < 1e-4


def test_near_tie_classifier_flags_planted_tie():
    s = np.array([[0.0, 5.0, 3.0, 3.0 + 1e-7, 1.0, 0.0]], np.float32)
    # sink 1, local 1 -> content = blocks 1..4; take 2 content -> boundary between 3.0 and 3.0+1e-7
    flags = O.selection_near_ties(s, np.array([4]), 1, 1, 1)
    assert flags[0]
    assert not O.selection_near_ties(s, np.array([3]), 1, 1, 1)[0]


def test_budget_near_half_flags():
    w = np.array([1.0, 1.0, 1.0, 1.0])
    # extra = 0.5 each -> lo + 0.5 exactly on the boundary
    assert O.budget_near_half(w, 6, 6.5).all()
    assert not O.budget_near_half(w, 6, 6.2).any()
