"""The eviction baselines (H2O, SnapKV) on the GPU against the NumPy oracle.

* key importance (adakv_key_importance): the reference's parity bar for its
  torch runtime (tests/test_baselines_runtime.py:45-61: max error / max
  importance < 1e-4) against the oracle's fp64 computation, for fp32, fp16 and
  bf16 prompts (16-bit inputs compared on their exact fp32 values), head_dim
  64 and 128, unexpanded grouped-query K, prompt lengths that are no multiple
  of the tiles, windows longer than the prompt; deterministic reruns; at 8K
  tokens the size-independent identity that the importances of a head add up
  to its number of queries.
* pool (adakv_importance_pool): bit-equal to the oracle's edge-clipped max.
* retained set (adakv_retain_blocks) on the oracle's own importance:
  bit-equal masks except heads whose last retained and first evicted block
  sums are within 1e-6 relative (counted, at most a few); sink/local forced,
  exact counts; the radix select's fallback path (more than 512 content
  blocks retained); end to end (HIP importance -> HIP retention) with the
  near-tie margin widened to the importance tolerance.
* tables: mask_to_block_table and frozen_decode_block_table restated from
  tests/test_baselines_runtime.py:124-172; the no-sync frozen_table equals the
  mask form.
* the reference's headline (tests/test_baselines.py:97-112): H2O and SnapKV
  evict a needle that is cold during the prompt, AdaKV's plan re-selects it;
  the frozen decode equals the oracle's frozen_sparse_attention.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from gpu_util import DEV, need_gpu, say, to_np, torch
from oracle import adakv_oracle as O

pytestmark = pytest.mark.gpu

DT = {"fp32": None, "fp16": None, "bf16": None}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    need_gpu()
    DT.update(fp32=torch.float32, fp16=torch.float16, bf16=torch.bfloat16)


def _BR():
    from adakv import baselines_rt
    return baselines_rt


def _qk(seed, Hq, Hkv, L, D, dtype, scale=0.5):
    rng = np.random.default_rng(seed)
    Q = (rng.standard_normal((Hq, L, D)) * scale).astype(np.float32)
    K = (rng.standard_normal((Hkv, L, D)) * scale).astype(np.float32)
    Qt = torch.from_numpy(Q).to(DEV, dtype)
    Kt = torch.from_numpy(K).to(DEV, dtype)
    # the oracle sees the exact values the GPU reads, K expanded to q-heads
    return to_np(Qt), O.expand_gqa(to_np(Kt), Hq), Qt, Kt


def _rel(got, want):
    return float(np.abs(got - want).max() / (np.abs(want).max() + 1e-30))


@pytest.mark.parametrize("dtype,D,Hq,Hkv,L", [
    ("fp32", 64, 6, 6, 384),          # tests/test_baselines_runtime.py:27-29 shapes
    ("fp32", 64, 6, 2, 203),
    ("bf16", 128, 8, 2, 1000),
    ("fp16", 128, 4, 4, 77),
    ("bf16", 64, 4, 1, 15),
    ("fp32", 128, 2, 1, 1),
    ("fp32", 64, 2, 1, 3000),         # few query waves: pass 1 splits the keys (3 ranges)
    ("bf16", 128, 4, 2, 5000),        # window: a 5-way key split
])
@pytest.mark.parametrize("window", [None, 32])
def test_importance_matches_oracle(dtype, D, Hq, Hkv, L, window):
    BR = _BR()
    say(f"importance {dtype} D={D} Hq={Hq} Hkv={Hkv} L={L} window={window}")
    Qn, Kn, Qt, Kt = _qk(L + D, Hq, Hkv, L, D, DT[dtype])
    first = 0 if window is None else L - min(window, L)
    got = BR.key_importance(Qt, Kt, first)
    again = BR.key_importance(Qt, Kt, first)
    torch.cuda.synchronize()
    want = O.key_importance(Qn, Kn, first)
    rel = _rel(to_np(got), want)
    say(f"  max err / max importance {rel:.2e}")
    assert rel < 1e-4
    assert torch.equal(got, again), "importance is not deterministic"


def test_importance_of_expanded_and_grouped_k_agree():
    BR = _BR()
    say("importance: K per KV head == K expanded to q-heads")
    _, _, Qt, Kt = _qk(3, 8, 2, 300, 128, torch.bfloat16)
    a = BR.h2o_key_importance_torch(Qt, Kt)
    b = BR.h2o_key_importance_torch(Qt, BR.expand_kv_heads(Kt, 4).contiguous())
    assert torch.equal(a, b)


def test_importance_strided_prompt_views():
    """HF hands q as a [B, Hq, L, D] view of [B, L, Hq, D] (token stride Hq*D)."""
    BR = _BR()
    say("importance on strided views")
    Qn, Kn, Qt, Kt = _qk(4, 4, 2, 130, 64, torch.float32)
    Qv = Qt.transpose(0, 1).contiguous().transpose(0, 1)
    Kv = Kt.transpose(0, 1).contiguous().transpose(0, 1)
    assert Qv.stride(1) == 4 * 64
    assert torch.equal(BR.key_importance(Qv, Kv, 0), BR.key_importance(Qt, Kt, 0))


@pytest.mark.parametrize("first", [0, 8192 - 32])
def test_importance_columns_add_up_to_the_query_count_at_8k(first):
    BR = _BR()
    say(f"importance at 8192 tokens (bf16, Llama-8B heads), first_query={first}")
    _, _, Qt, Kt = _qk(5, 32, 8, 8192, 128, torch.bfloat16)
    imp = BR.key_importance(Qt, Kt, first)
    torch.cuda.synchronize()
    tot = imp.double().sum(dim=1)
    err = float(((tot - (8192 - first)).abs() / (8192 - first)).max())
    say(f"  max rel error of the column total {err:.2e}")
    assert err < 1e-4 and bool((imp >= 0).all()) and bool(torch.isfinite(imp).all())
    # the last key is seen by the last query only: its softmax weight there
    q, k = Qt[:, -1].float(), BR.expand_kv_heads(Kt, 4).float()
    lg = torch.einsum("hd,hjd->hj", q, k) / math.sqrt(128)
    p_last = torch.softmax(lg.double(), dim=1)[:, -1]
    assert float((imp[:, -1].double() - p_last).abs().max()) < 1e-5


@pytest.mark.parametrize("kernel", [3, 7, 9])
def test_pool_matches_oracle(kernel):
    BR = _BR()
    say(f"pool kernel {kernel}")
    x = np.random.default_rng(kernel).random((5, 1000)).astype(np.float32)
    got = BR.importance_pool(torch.from_numpy(x).to(DEV), kernel)
    np.testing.assert_array_equal(to_np(got), O.maxpool_same(x, kernel))


def test_snapkv_importance_matches_oracle():
    BR = _BR()
    say("snapkv importance (window 32, pool 7)")
    Qn, Kn, Qt, Kt = _qk(6, 6, 6, 384, 64, torch.float32)
    got = BR.snapkv_key_importance_torch(Qt, Kt, 32, 7)
    assert _rel(to_np(got), O.snapkv_key_importance(Qn, Kn, 32, 7)) < 1e-4


def _check_retain(imp, bs, n_real, budget, sink, local, cmin, tol=1e-6, max_excl=2):
    BR = _BR()
    mask, table, lens = BR.retain_blocks_table(torch.from_numpy(imp).to(DEV), bs, n_real, budget, sink, local, cmin)
    want = O.retain_blocks(imp, bs, n_real, budget, sink, local, cmin)
    got = to_np(mask).astype(bool)
    nb = want.shape[1]
    k = min(max(budget, min(min(sink, nb) + min(local, nb) + cmin, nb)), nb)
    assert got.shape == want.shape
    assert (got.sum(axis=1) == k).all(), got.sum(axis=1)
    assert got[:, :min(sink, nb)].all() and got[:, nb - min(local, nb):].all()
    lens_np = lens.cpu().numpy()
    assert (lens_np == k).all()
    tab = table.cpu().numpy()
    for h in range(got.shape[0]):
        assert tab[h].tolist() == np.flatnonzero(got[h]).tolist(), "table is not the ascending mask"
    ties = O.retain_near_ties(imp, bs, n_real, budget, sink, local, cmin, rel_tol=tol)
    bad = [h for h in range(got.shape[0]) if not ties[h] and not np.array_equal(got[h], want[h])]
    assert not bad, f"heads {bad} differ from the oracle"
    assert int(ties.sum()) <= max_excl, f"{int(ties.sum())} near-tie heads excluded"
    return int(ties.sum())


@pytest.mark.parametrize("bs,n_real,budget,sink,local,cmin", [
    (16, 384, 6, 1, 2, 1), (16, 384, 8, 1, 2, 1), (16, 384, 12, 1, 2, 1),
    (16, 383, 8, 1, 4, 1),              # partial tail block
    (16, 5000, 64, 2, 4, 3),
    (32, 40000, 1000, 1, 4, 1),         # > 512 content blocks: the select's fallback path
    (16, 262144, 8, 1, 4, 1),           # 16384 blocks: the kernel's limit
    (16, 40, 100, 1, 4, 1),             # budget above nb: every block
    (16, 16, 1, 1, 1, 1),               # a single block
])
def test_retain_matches_oracle_on_the_same_importance(bs, n_real, budget, sink, local, cmin):
    say(f"retain bs={bs} n_real={n_real} budget={budget} sink={sink} local={local} c_min={cmin}")
    rng = np.random.default_rng(n_real)
    imp = (rng.random((6, n_real)) * rng.random((6, 1)) * 4).astype(np.float32)
    n = _check_retain(imp, bs, n_real, budget, sink, local, cmin)
    say(f"  near-tie heads excluded: {n}")


def test_retain_ties_take_lower_blocks():
    say("retain: equal block sums")
    imp = np.zeros((3, 160), dtype=np.float32)
    _check_retain(imp, 16, 160, 4, 1, 1, 1, max_excl=3)
    got = _BR().retain_blocks_torch(torch.from_numpy(imp).to(DEV), 16, 160, 4, 1, 1, 1)
    assert np.flatnonzero(to_np(got)[0]).tolist() == [0, 1, 2, 9]


@pytest.mark.parametrize("which", ["h2o", "snapkv"])
@pytest.mark.parametrize("budget", [6, 8, 12])
def test_retained_masks_end_to_end(which, budget):
    # tests/test_baselines_runtime.py:64-86 (agreement > 0.99 there; exact here
    # outside near-ties at the importance tolerance)
    BR = _BR()
    say(f"{which} retained mask end to end, budget {budget}")
    for seed in (0, 1, 2):
        Qn, Kn, Qt, Kt = _qk(seed, 6, 6, 384, 64, torch.float32)
        if which == "h2o":
            got = BR.h2o_retained_mask_torch(Qt, Kt, 16, budget, 1, 2, 1)
            imp = O.h2o_key_importance(Qn, Kn)
        else:
            got = BR.snapkv_retained_mask_torch(Qt, Kt, 16, budget, 32, 7, 1, 2, 1)
            imp = O.snapkv_key_importance(Qn, Kn, 32, 7)
        want = O.retain_blocks(imp, 16, 384, budget, 1, 2, 1)
        ties = O.retain_near_ties(imp, 16, 384, budget, 1, 2, 1, rel_tol=2e-4)
        g = to_np(got).astype(bool)
        for h in range(6):
            if not ties[h]:
                assert np.array_equal(g[h], want[h]), f"seed {seed} head {h}"
        assert (g.sum(axis=1) == min(max(budget, 4), 24)).all()


def test_mask_to_block_table():
    # tests/test_baselines_runtime.py:124-135
    BR = _BR()
    say("mask_to_block_table")
    _, _, Qt, Kt = _qk(4, 6, 6, 384, 64, torch.float32)
    m = BR.h2o_retained_mask_torch(Qt, Kt, 16, 8, 1, 2, 1)
    bt, sl = BR.mask_to_block_table(m)
    assert bt.shape == (6, 8) and bt.dtype == torch.int32 and bool((sl == 8).all())
    for h in range(6):
        assert torch.equal(bt[h], torch.nonzero(m[h]).flatten().to(torch.int32))
    uneven = m.clone()
    uneven[0, 5] = ~uneven[0, 5]
    with pytest.raises(AssertionError):
        BR.mask_to_block_table(uneven)


@pytest.mark.parametrize("grow", [0, 1, 3, 10])
def test_frozen_decode_block_table(grow):
    # tests/test_baselines_runtime.py:147-172
    BR = _BR()
    say(f"frozen decode table, {grow} new blocks")
    SINK, LOCAL = 1, 2
    _, _, Qt, Kt = _qk(5, 6, 6, 384, 64, torch.float32)
    imp = BR.h2o_key_importance_torch(Qt, Kt)
    fmask, ftab, flens = BR.retain_blocks_table(imp, 16, 384, 8, SINK, LOCAL, 1)
    nbp = fmask.shape[1]
    nb_now = nbp + grow
    bt, sl = BR.frozen_decode_block_table(fmask, nb_now, SINK, LOCAL)
    dm = torch.zeros(6, nb_now, dtype=torch.bool, device=DEV)
    dm.scatter_(1, bt.long(), True)
    want = torch.from_numpy(O.frozen_decode_mask(to_np(fmask).astype(bool), nb_now, SINK, LOCAL)).to(DEV)
    assert torch.equal(dm, want)
    assert torch.equal(dm[:, SINK:nbp - LOCAL], fmask[:, SINK:nbp - LOCAL])
    assert bool(dm[:, nb_now - LOCAL:].all()) and bool((sl == 8 + min(LOCAL, grow)).all())
    t2, l2 = BR.frozen_table(ftab, flens, nbp, nb_now, SINK, LOCAL)
    assert torch.equal(l2, sl)
    assert torch.equal(t2[:, :int(sl[0])], bt)
    with pytest.raises(AssertionError):
        BR.frozen_decode_block_table(fmask, nbp - 1, SINK, LOCAL)


def _cold_needle(seed):
    # tests/test_baselines.py:35-48
    H, S, D, BS, NEEDLE = 4, 512, 64, 16, 20
    rng = np.random.default_rng(seed)
    r = rng.standard_normal(D)
    r = (r / (np.linalg.norm(r) + 1e-9)).astype(np.float32)
    K = (rng.standard_normal((H, S, D)) * 0.1).astype(np.float32)
    V = rng.standard_normal((H, S, D)).astype(np.float32)
    K[:, NEEDLE * BS:(NEEDLE + 1) * BS] = r[None, None, :] * 30.0
    Q = rng.standard_normal((H, S, D)).astype(np.float32)
    Q = Q - (Q @ r)[..., None] * r[None, None, :]
    return Q, K, V, np.broadcast_to(r, (H, D)).astype(np.float32).copy()


def test_eviction_loses_the_cold_needle_adakv_keeps_it():
    from adakv_amd import ops
    BR = _BR()
    say("cold needle: H2O / SnapKV evict, AdaKV re-selects")
    Q, K, V, q = _cold_needle(0)
    Qt, Kt, Vt, qt = (torch.from_numpy(x).to(DEV) for x in (Q, K, V, q))
    h2o = BR.h2o_retained_mask_torch(Qt, Kt, 16, 8, 1, 2, 1)
    snap = BR.snapkv_retained_mask_torch(Qt, Kt, 16, 8, 32, 7, 1, 2, 1)
    c = ops.centroid_build(Kt[None], 16)
    table, lens = ops.plan(qt[None], c, 16, ops.BudgetParams(avg_budget=8, k_min=1, k_max=32, n_sink_blocks=1,
                                                             n_local_blocks=2, c_min=1,
                                                             budget_policy="fixed"))
    ada = [set(table[0, h, :int(lens[0, h])].tolist()) for h in range(4)]
    assert not bool(h2o[:, 20].any()) and not bool(snap[:, 20].any())
    assert all(20 in s for s in ada)


def test_frozen_decode_matches_oracle_frozen_attention():
    from adakv_amd import ops
    BR = _BR()
    say("frozen decode output vs oracle frozen_sparse_attention")
    Q, K, V, q = _cold_needle(1)
    Qt, Kt, Vt, qt = (torch.from_numpy(x).to(DEV) for x in (Q, K, V, q))
    mask, table, lens = BR.retain_blocks_table(BR.h2o_key_importance_torch(Qt, Kt), 16, 512, 8, 1, 2, 1)
    out = ops.sparse_decode(qt[None], Kt[None], Vt[None], table[None].contiguous(), lens[None].contiguous(), 16)
    want, counts = O.frozen_sparse_attention(q, K, V, to_np(mask).astype(bool), 16)
    assert (counts == 8).all()
    rel = np.linalg.norm(to_np(out[0]) - want) / np.linalg.norm(want)
    say(f"  rel L2 {rel:.2e}")
    assert rel < 1e-5
    dense = O.dense_attention(q, K, V)
    assert np.linalg.norm(want - dense) / np.linalg.norm(dense) > 0.1   # the evicted needle mattered


def test_argument_errors():
    BR = _BR()
    say("eviction argument errors")
    x = torch.zeros(2, 64, device=DEV)
    with pytest.raises(ValueError):
        BR.importance_pool(x, 4)
    q = torch.zeros(4, 64, 64, device=DEV)
    with pytest.raises(ValueError):
        BR.key_importance(q, torch.zeros(3, 64, 64, device=DEV))          # 4 % 3
    with pytest.raises(ValueError):
        BR.key_importance(q, torch.zeros(2, 64, 64, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        BR.key_importance(torch.zeros(4, 64, 96, device=DEV), torch.zeros(2, 64, 96, device=DEV))   # head_dim 96
    with pytest.raises(ValueError):
        BR.retain_blocks_torch(torch.zeros(2, 16 * 16385, device=DEV), 16, 16 * 16385, 8)           # > 16384 blocks
