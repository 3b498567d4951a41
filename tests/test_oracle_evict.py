"""Oracle checks for the eviction baselines (H2O, SnapKV).

The restatement in oracle/adakv_oracle.py (key_importance, maxpool_same,
retain_blocks, frozen_decode_mask, frozen_sparse_attention) is pinned here by
what mathematics fixes -- every softmax row sums to one, so the importances of
all keys add up to the number of queries; the last key is seen by the last
query only; a pure-Python brute force on tiny inputs; SciPy's
maximum_filter1d for the pool; a sort for the retained set -- and by the
reference's own CPU tests (tests/test_baselines.py, tests/test_baselines_runtime.py)
restated against the oracle.  Plausible mistakes planted in copies of the
oracle (no causal mask, the wrong softmax axis or scale, a pool without edge
clipping) each fail one of the pins.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import adakv_oracle as O

BS = 16
H, S, D = 4, 512, 64
NB = S // BS
SINK, LOCAL, CMIN = 1, 2, 1
FLOOR = SINK + LOCAL + CMIN
NEEDLE = 20


def _unit(rng, d):
    v = rng.standard_normal(d)
    return (v / (np.linalg.norm(v) + 1e-9)).astype(np.float32)


def _cold_needle_case(seed=0):
    # tests/test_baselines.py:35-48: a needle block that the prompt's queries
    # never look at (their component along it is projected out) but the decode
    # query points straight at
    rng = np.random.default_rng(seed)
    r = _unit(rng, D)
    K = (rng.standard_normal((H, S, D)) * 0.1).astype(np.float32)
    V = rng.standard_normal((H, S, D)).astype(np.float32)
    K[:, NEEDLE * BS:(NEEDLE + 1) * BS] = r[None, None, :] * 30.0
    Q = rng.standard_normal((H, S, D)).astype(np.float32)
    Q = Q - (Q @ r)[..., None] * r[None, None, :]
    return Q, K, V, np.broadcast_to(r, (H, D)).astype(np.float32).copy()


def _qk(seed, H=3, S=96, D=16, scale=0.5):
    rng = np.random.default_rng(seed)
    return ((rng.standard_normal((H, S, D)) * scale).astype(np.float32),
            (rng.standard_normal((H, S, D)) * scale).astype(np.float32))


# ---- importance -------------------------------------------------------------
def _brute_importance(Q, K, first):
    Hh, Ss, Dd = K.shape
    out = np.zeros((Hh, Ss))
    for h in range(Hh):
        for i in range(first, Ss):
            logits = [sum(float(Q[h, i, d]) * float(K[h, j, d]) for d in range(Dd)) / math.sqrt(Dd)
                      for j in range(i + 1)]
            m = max(logits)
            e = [math.exp(x - m) for x in logits]
            z = sum(e)
            for j in range(i + 1):
                out[h, j] += e[j] / z
    return out


@pytest.mark.parametrize("first", [0, 5, 11])
def test_importance_brute_force(first):
    Q, K = _qk(1, H=2, S=12, D=5, scale=1.0)
    got = O.key_importance(Q, K, first)
    assert got.dtype == np.float32
    np.testing.assert_allclose(got, _brute_importance(Q, K, first), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("first", [0, 64, 95])
def test_importance_columns_add_up_to_the_query_count(first):
    Q, K = _qk(2)
    imp = O.key_importance(Q, K, first).astype(np.float64)
    np.testing.assert_allclose(imp.sum(axis=1), 96 - first, rtol=1e-6)
    assert (imp > 0).all() and np.isfinite(imp).all()


def test_last_key_is_seen_by_the_last_query_only():
    Q, K = _qk(3)
    imp = O.h2o_key_importance(Q, K)
    lg = np.einsum("hd,hjd->hj", Q[:, -1].astype(np.float64), K.astype(np.float64)) / math.sqrt(16)
    p = np.exp(lg - lg.max(axis=1, keepdims=True))
    np.testing.assert_allclose(imp[:, -1], p[:, -1] / p.sum(axis=1), rtol=1e-6)


def test_snapkv_is_the_pooled_window_importance():
    Q, K = _qk(4)
    raw = O.key_importance(Q, K, 96 - 32)
    np.testing.assert_array_equal(O.snapkv_key_importance(Q, K, 32, 7), O.maxpool_same(raw, 7))
    # a window longer than the prompt covers every query
    np.testing.assert_array_equal(O.snapkv_key_importance(Q, K, 500, 1), O.h2o_key_importance(Q, K))


@pytest.mark.parametrize("kernel", [1, 3, 7, 9])
def test_maxpool_matches_scipy_nearest(kernel):
    from scipy.ndimage import maximum_filter1d
    x = np.random.default_rng(5).standard_normal((3, 41)).astype(np.float32)
    np.testing.assert_array_equal(O.maxpool_same(x, kernel), maximum_filter1d(x, size=kernel, axis=1, mode="nearest"))


# ---- planted mistakes fail a pin ----------------------------------------------
def _mutant_importance(Q, K, first, causal=True, axis=-1, scale=None):
    Hh, Ss, Dd = K.shape
    lg = np.einsum("hid,hjd->hij", Q[:, first:].astype(np.float64), K.astype(np.float64))
    lg *= (1.0 / math.sqrt(Dd)) if scale is None else scale
    if causal:
        lg = np.where(np.arange(Ss)[None, :] <= np.arange(first, Ss)[:, None], lg, -np.inf)
    e = np.exp(lg - lg.max(axis=axis, keepdims=True))
    return (e / e.sum(axis=axis, keepdims=True)).sum(axis=1).astype(np.float32)


def _pins_hold(fn):
    Qs, Ks = _qk(1, H=2, S=12, D=5, scale=1.0)
    Q, K = _qk(3)
    try:
        np.testing.assert_allclose(fn(Qs, Ks, 0), _brute_importance(Qs, Ks, 0), rtol=2e-6, atol=1e-7)
        np.testing.assert_allclose(fn(Q, K, 40).astype(np.float64).sum(axis=1), 56, rtol=1e-6)
    except AssertionError:
        return False
    return True


def test_pins_reject_planted_importance_mistakes():
    assert _pins_hold(O.key_importance)
    assert not _pins_hold(lambda Q, K, f: _mutant_importance(Q, K, f, causal=False))
    assert not _pins_hold(lambda Q, K, f: _mutant_importance(Q, K, f, axis=1))
    assert not _pins_hold(lambda Q, K, f: _mutant_importance(Q, K, f, scale=1.0 / K.shape[2]))


def test_pins_reject_a_pool_without_edge_clipping():
    from scipy.ndimage import maximum_filter1d
    x = np.random.default_rng(6).standard_normal((2, 20)).astype(np.float32)
    wrap = np.stack([np.array([np.max(np.take(r, range(t - 3, t + 4), mode="wrap")) for t in range(20)]) for r in x])
    assert not np.array_equal(wrap, maximum_filter1d(x, size=7, axis=1, mode="nearest"))


# ---- retention ----------------------------------------------------------------
@pytest.mark.parametrize("budget", [1, 6, 8, 12, NB])
def test_retain_exact_budget_forced_blocks_and_top_sums(budget):
    rng = np.random.default_rng(7)
    imp = rng.random((H, S)).astype(np.float32)
    m = O.retain_blocks(imp, BS, S, budget, SINK, LOCAL, CMIN)
    k = min(max(budget, FLOOR), NB)
    assert m.shape == (H, NB) and (m.sum(axis=1) == k).all()
    assert m[:, :SINK].all() and m[:, NB - LOCAL:].all()
    sums = imp.reshape(H, NB, BS).astype(np.float64).sum(axis=2)
    for h in range(H):
        content = sorted(range(SINK, NB - LOCAL), key=lambda b: -sums[h, b])
        want = set(range(SINK)) | set(range(NB - LOCAL, NB)) | set(content[:k - SINK - LOCAL])
        assert set(np.flatnonzero(m[h])) == want


def test_retain_partial_tail_block_and_ties():
    imp = np.ones((2, 37), dtype=np.float32)             # 3 blocks of 16: the last holds 5 tokens
    blk = O.retain_block_sums(imp, 16, 37)
    assert blk.tolist() == [[16.0, 16.0, 5.0]] * 2
    flat = np.zeros((1, 160), dtype=np.float32)          # all content sums tie: lowest blocks first
    m = O.retain_blocks(flat, 16, 160, 4, 1, 1, 1)
    assert np.flatnonzero(m[0]).tolist() == [0, 1, 2, 9]


def test_retain_near_ties_flags_only_close_boundaries():
    imp = np.zeros((2, 8 * 16), dtype=np.float32)
    imp[:, 16:32] = 1.0                                   # block 1
    imp[0, 32:48] = 1.0                                   # head 0: block 2 ties block 1
    imp[1, 32:48] = 0.5
    flags = O.retain_near_ties(imp, 16, 128, 4, 1, 2, 1)  # one content block retained
    assert flags.tolist() == [True, False]


# ---- the reference's CPU scenarios (tests/test_baselines.py) --------------------
def test_eviction_loses_the_cold_needle_adakv_keeps_it():
    Q, K, V, q_dec = _cold_needle_case(0)
    h2o = O.retain_blocks(O.h2o_key_importance(Q, K), BS, S, 8, SINK, LOCAL, CMIN)
    snap = O.retain_blocks(O.snapkv_key_importance(Q, K), BS, S, 8, SINK, LOCAL, CMIN)
    _, _, ada = O.sparse_attention(q_dec, K, V, block_size=BS, avg_budget=8, k_min=1, k_max=NB,
                                   n_sink_blocks=SINK, n_local_blocks=LOCAL, c_min=CMIN,
                                   budget_policy="fixed", return_mask=True)
    assert not h2o[:, NEEDLE].any() and not snap[:, NEEDLE].any() and ada[:, NEEDLE].all()


def test_h2o_keeps_the_prompt_heavy_hitter():
    rng = np.random.default_rng(3)
    K = (rng.standard_normal((H, S, D)) * 0.1).astype(np.float32)
    hot, d = 11, _unit(rng, D)
    K[:, hot * BS:(hot + 1) * BS] = d[None, None, :] * 30.0
    Q = np.broadcast_to(d, (H, S, D)).astype(np.float32).copy()
    assert O.retain_blocks(O.h2o_key_importance(Q, K), BS, S, 6, SINK, LOCAL, CMIN)[:, hot].all()


def test_frozen_attention_full_set_is_dense_evicted_needle_is_not():
    Q, K, V, q_dec = _cold_needle_case(1)
    dense = O.dense_attention(q_dec, K, V)
    h2o = O.retain_blocks(O.h2o_key_importance(Q, K), BS, S, 8, SINK, LOCAL, CMIN)
    ev, counts = O.frozen_sparse_attention(q_dec, K, V, h2o, BS)
    full, _ = O.frozen_sparse_attention(q_dec, K, V, np.ones((H, NB), dtype=bool), BS)
    assert (counts == 8).all()
    assert np.linalg.norm(full - dense) / np.linalg.norm(dense) < 1e-5
    assert np.linalg.norm(ev - dense) / np.linalg.norm(dense) > 0.1


def test_frozen_decode_mask_tracks_the_tail():
    # tests/test_baselines_runtime.py:147-172
    Q, K = _qk(5, H=6, S=384, D=64)
    f = O.retain_blocks(O.h2o_key_importance(Q, K), BS, 384, 8, SINK, LOCAL, CMIN)
    nbp = f.shape[1]
    assert np.array_equal(O.frozen_decode_mask(f, nbp, SINK, LOCAL), f)
    m = O.frozen_decode_mask(f, nbp + 3, SINK, LOCAL)
    assert np.array_equal(m[:, SINK:nbp - LOCAL], f[:, SINK:nbp - LOCAL])
    assert m[:, -LOCAL:].all() and (m.sum(axis=1) == 8 + LOCAL).all()
    with pytest.raises(AssertionError):
        O.frozen_decode_mask(f, nbp - 1, SINK, LOCAL)
