"""The minmax (Quest) estimator on the GPU, through the C ABI
(adakv/estimator.py:50-57,76-79, adakv/attention.py:131-138,190-198).

* summaries: the per-dimension max and min of every block's real keys,
  bit-exact against the oracle (both are exact in the key type and in fp32),
  after a build, after token-by-token appends and after a multi-token append;
* scores: the Quest bound max(q,0) . kmax + min(q,0) . kmin against an fp64
  evaluation, within the fp32 accumulation bound;
* selection: the reference's golden mask and counts of its minmax case, and
  the oracle's budget and selection run on the GPU's own summaries for bf16 /
  fp16 decode steps (the Quest cell, fixed budget, and the budget-only
  ablation, adaptive budget: adakv/attention.py:166-171), near-ties excluded;
* output: fp64 attention over the GPU's own selection, bf16 tolerance;
* the Python API: AdaKVCache(estimator="minmax") and plan_selection mirror the
  reference's factorial test (tests/test_factorial_selection.py:42-108).
"""
from __future__ import annotations

import numpy as np
import pytest

import cases
import golden_check
from gpu_util import DEV, compare_selection, need_gpu, say, torch
from oracle import adakv_oracle as O
from test_gpu_fused import _inputs, _params, _run

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    need_gpu()


def _ops():
    from adakv_amd import ops
    return ops


def _split(c: torch.Tensor, D: int):
    c = c.float().cpu().numpy()
    return c[..., :D], c[..., D:]


# ------------------------------------------------------------------ summaries
@pytest.mark.parametrize("kdt,cdt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.float16, torch.float16), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("S,D,bs", [(4001, 64, 16), (37, 128, 5), (1000, 32, 32)])
def test_minmax_build_bit_exact(kdt, cdt, S, D, bs):
    ops = _ops()
    say(f"minmax build {kdt}->{cdt} S={S} D={D} bs={bs}")
    rng = np.random.RandomState(S + D)
    K = torch.from_numpy(rng.standard_normal((1, 3, S, D)).astype(np.float32)).to(kdt)
    c = ops.centroid_build(K.to(DEV), bs, centroid_dtype=cdt, estimator="minmax")
    torch.cuda.synchronize()
    assert c.shape == (1, 3, ops.n_blocks(S, bs), 2 * D) and c.dtype == cdt
    ref = O.build_block_summaries(K[0].float().numpy(), bs, kind="minmax")
    kmax, kmin = _split(c[0], D)
    assert np.array_equal(kmax, ref["kmax"]) and np.array_equal(kmin, ref["kmin"])


def test_minmax_build_ragged_batch():
    """Per-sequence lengths: rows of each sequence's own blocks only (a partial
    last block's padding never enters the bounds, adakv/attention.py:131-134)."""
    ops = _ops()
    say("minmax build ragged [1, 777, 4096]")
    rng = np.random.RandomState(5)
    lens = [1, 777, 4096]
    K = torch.from_numpy(rng.standard_normal((3, 2, 4096, 64)).astype(np.float32)).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    c = ops.centroid_build(K.to(DEV), 16, seq_lens=sl, estimator="minmax")
    torch.cuda.synchronize()
    for b, L in enumerate(lens):
        ref = O.build_block_summaries(K[b, :, :L].float().numpy(), 16, kind="minmax")
        nb = ref["kmax"].shape[1]
        kmax, kmin = _split(c[b, :, :nb], 64)
        assert np.array_equal(kmax, ref["kmax"]) and np.array_equal(kmin, ref["kmin"])
        assert (c[b, :, nb:] == 0).all()


def test_minmax_append_equals_rebuild():
    ops = _ops()
    say("minmax append vs rebuild")
    rng = np.random.RandomState(6)
    Hkv, S0, D, bs, steps = 4, 100, 64, 16, 50
    K = torch.from_numpy(rng.standard_normal((1, Hkv, S0 + steps, D)).astype(np.float32)).to(DEV)
    cap = ops.n_blocks(S0 + steps, bs) + 3
    c = ops.centroid_build(K[:, :, :S0], bs, max_blocks=cap, estimator="minmax")
    for t in range(steps):
        ops.centroid_append(K[:, :, : S0 + t + 1], c, bs, n_new=1)
    c2 = ops.centroid_build(K, bs, max_blocks=cap, estimator="minmax")
    ops.centroid_append(K, c2, bs, n_new=37)      # multi-token append spanning blocks
    torch.cuda.synchronize()
    ref = O.build_block_summaries(K[0].cpu().numpy(), bs, kind="minmax")
    nb = ref["kmax"].shape[1]
    for cc in (c, c2):
        kmax, kmin = _split(cc[0, :, :nb], D)
        assert np.array_equal(kmax, ref["kmax"]) and np.array_equal(kmin, ref["kmin"])


# --------------------------------------------------------------------- scores
@pytest.mark.parametrize("qdt,cdt,D,G", [(torch.bfloat16, torch.bfloat16, 128, 4),
                                         (torch.float16, torch.float16, 64, 8),
                                         (torch.float32, torch.float32, 128, 4),
                                         (torch.float32, torch.bfloat16, 32, 2),
                                         (torch.bfloat16, torch.float32, 64, 1)])
def test_minmax_scores_quest_bound(qdt, cdt, D, G):
    """Scores vs fp64 max(q,0).kmax + min(q,0).kmin on the GPU's own bounds.
    With q in fp32 and 16-bit bounds the matrix cores take q rounded to the
    bounds' type (as for centroids), so the reference uses that q."""
    ops = _ops()
    say(f"minmax scores q {qdt} bounds {cdt} D={D} G={G}")
    rng = np.random.RandomState(D + G)
    Hkv, S, bs = 4, 5000, 16
    kdt = cdt if cdt != torch.float32 else qdt
    K = torch.from_numpy(rng.standard_normal((1, Hkv, S, D)).astype(np.float32)).to(kdt).to(DEV)
    q = torch.from_numpy(rng.standard_normal((1, Hkv * G, D)).astype(np.float32)).to(qdt).to(DEV)
    c = ops.centroid_build(K, bs, centroid_dtype=cdt, estimator="minmax")
    sc = ops.block_scores(q, c, bs, seq_len=S)
    torch.cuda.synchronize()
    nb = ops.n_blocks(S, bs)
    qq = q[0].to(cdt).double() if qdt == torch.float32 and cdt != torch.float32 else q[0].double()
    qn = qq.cpu().numpy()
    kmax, kmin = (O.expand_gqa(x.astype(np.float64), Hkv * G) for x in _split(c[0, :, :nb], D))
    qp, qm = np.maximum(qn, 0)[:, None, :], np.minimum(qn, 0)[:, None, :]
    ref = (qp * kmax + qm * kmin).sum(-1)
    bound = (np.abs(qp) * np.abs(kmax) + np.abs(qm) * np.abs(kmin)).sum(-1)
    got = sc[0, :, :nb].double().cpu().numpy()
    assert np.all(np.abs(got - ref) <= 3e-5 * bound + 1e-30)


# ------------------------------------------------------------------ selection
def test_minmax_plan_matches_reference_golden():
    """fp32 path vs the reference's own scores, mask and counts (minmax_fixed)."""
    ops = _ops()
    name = "minmax_fixed"
    say(f"minmax plan golden {name}")
    p = cases.params(name)
    q, Kkv, Vkv = cases.make_inputs(name)
    g = golden_check.load(name)
    bs = p["bs"]
    budget = ops.BudgetParams(avg_budget=p["avg"], k_min=p["kmin"], k_max=p["kmax"],
                              n_sink_blocks=p["sink"], n_local_blocks=p["local"], c_min=p["cmin"],
                              budget_policy=p["policy"])
    k = torch.from_numpy(Kkv).to(DEV).unsqueeze(0)
    c = ops.centroid_build(k, bs, estimator="minmax")
    qt = torch.from_numpy(q).to(DEV).unsqueeze(0)
    sc = ops.block_scores(qt, c, bs, seq_len=Kkv.shape[1])
    table, lens = ops.plan(qt, c, bs, budget, seq_len=Kkv.shape[1], estimator="minmax")
    torch.cuda.synchronize()
    nb = g["scores"].shape[1]
    scale = float(np.abs(g["scores"]).max())
    assert np.abs(sc[0, :, :nb].cpu().numpy() - g["scores"]).max() <= 1e-5 * scale
    table, lens = table[0].cpu().numpy(), lens[0].cpu().numpy()
    lo, _, target, _ = O.budget_bounds(nb, p["avg"], p["kmin"], p["kmax"], p["sink"], p["local"], p["cmin"])
    excl = compare_selection(g["scores"], table, lens, k_oracle=g["k"], w_oracle=np.ones(q.shape[0]),
                             lo=lo, target=target, sink=p["sink"], local=p["local"], cmin=p["cmin"],
                             policy=p["policy"])
    say(f"  {excl} heads excluded as near-ties")
    if excl == 0:
        gm = np.zeros_like(g["mask"])
        for h in range(table.shape[0]):
            gm[h, table[h, : lens[h]]] = True
        assert np.array_equal(gm, g["mask"])
        assert np.array_equal(lens, g["counts"])


def test_minmax_fused_step_matches_reference_golden_output():
    """fp32 decode step with minmax scoring vs the reference's sparse_attention output."""
    ops = _ops()
    name = "minmax_fixed"
    say(f"minmax fused golden {name}")
    p = cases.params(name)
    q, Kkv, Vkv = cases.make_inputs(name)
    g = golden_check.load(name)
    bs = p["bs"]
    budget = ops.BudgetParams(avg_budget=p["avg"], k_min=p["kmin"], k_max=p["kmax"],
                              n_sink_blocks=p["sink"], n_local_blocks=p["local"], c_min=p["cmin"],
                              budget_policy=p["policy"])
    k = torch.from_numpy(Kkv).to(DEV).unsqueeze(0)
    v = torch.from_numpy(Vkv).to(DEV).unsqueeze(0)
    c = ops.centroid_build(k, bs, estimator="minmax")
    out, table, lens = ops.decode_fused(torch.from_numpy(q).to(DEV).unsqueeze(0), k, v, c, bs, budget,
                                        return_selection=True, estimator="minmax")
    torch.cuda.synchronize()
    table, lens, got = table[0].cpu().numpy(), lens[0].cpu().numpy(), out[0].cpu().numpy()
    same = np.array([set(table[h, : lens[h]].tolist()) == set(np.flatnonzero(g["mask"][h]).tolist())
                     for h in range(q.shape[0])])
    assert same.mean() >= 0.75
    assert np.abs(got[same] - g["out"][same]).max() <= 2e-4
    ref = O.ref_from_table(q, Kkv, Vkv, table, lens, bs, q.shape[0] // Kkv.shape[0])
    assert np.abs(got - ref).max() <= 2e-4


GOLDEN_INPUTS = ["minmax_fixed", "cfg1_seed0", "partial_tail", "gqa6_kmax256", "bs32", "tiny_overlap",
                 "single_block", "planted"]


@pytest.mark.parametrize("policy", ["fixed", "adaptive"])
@pytest.mark.parametrize("name", GOLDEN_INPUTS)
def test_minmax_fused_bf16_golden_inputs(name, policy):
    p = cases.params(name)
    p.update(est="minmax", policy=policy)
    say(f"minmax fused bf16 {name} {policy}")
    q, K, V = cases.make_inputs(name)
    _run(q[None], K[None], V[None], p, p["bs"], torch.bfloat16)


def test_minmax_fused_fp16():
    p = cases.params("minmax_fixed")
    say("minmax fused fp16 minmax_fixed")
    q, K, V = cases.make_inputs("minmax_fixed")
    _run(q[None], K[None], V[None], p, p["bs"], torch.float16)


@pytest.mark.parametrize("Hq,Hkv,D", [(64, 8, 64), (40, 5, 128), (16, 16, 32)])
def test_minmax_fused_many_heads(Hq, Hkv, D):
    say(f"minmax fused Hq={Hq} Hkv={Hkv} D={D}")
    q, K, V = _inputs(31, 1, Hq, Hkv, 4096, D)
    _run(q, K, V, _params(avg=10, est="minmax"), 16, torch.bfloat16)


@pytest.mark.parametrize("bs", [24, 8])
def test_minmax_fused_block_sizes(bs):
    say(f"minmax fused block size {bs}")
    q, K, V = _inputs(32, 1, 16, 4, 3001, 128)
    _run(q, K, V, _params(avg=12, est="minmax", policy="fixed"), bs, torch.bfloat16)


def test_minmax_fused_append_several_rows():
    """append_new spanning three blocks: their bounds are recomputed from K by the step."""
    say("minmax fused append 40 tokens")
    q, K, V = _inputs(33, 1, 32, 8, 4096 + 7, 128)
    _run(q, K, V, _params(avg=8, est="minmax"), 16, torch.bfloat16, append_new=40, corrupt_tail=40)


def test_minmax_fused_ragged_batch():
    say("minmax fused ragged batch [0, 1, 777, 4096]")
    q, K, V = _inputs(34, 4, 16, 4, 4096, 128)
    _run(q, K, V, _params(avg=8, est="minmax", policy="fixed"), 16, torch.bfloat16,
         seq_lens=[0, 1, 777, 4096])


# ------------------------------------------------------------------ Python API
def _factorial_fixture(seed=0):
    # tests/test_factorial_selection.py:19-34: HKV 2, S 320, D 64, group 6, block 16
    rng = np.random.RandomState(seed)
    k = torch.from_numpy(rng.standard_normal((2, 320, 64)).astype(np.float32)).to(DEV)
    v = torch.from_numpy(rng.standard_normal((2, 320, 64)).astype(np.float32)).to(DEV)
    q = torch.from_numpy(rng.standard_normal((12, 64)).astype(np.float32)).to(DEV)
    return q, k, v


def test_minmax_cache_and_factorial_cells():
    """AdaKVCache(estimator="minmax") holds centroids and exact bounds; every
    (estimator, policy) cell runs, keeps >= c_min content blocks per head,
    honours a fixed budget and agrees with the oracle's mask
    (tests/test_factorial_selection.py:42-108)."""
    from adakv.attention import AdaKVCache, plan_selection
    say("minmax cache + factorial cells")
    q, k, v = _factorial_fixture()
    cc = AdaKVCache(16, "centroid").append_prefill(k, v)
    cm = AdaKVCache(16, "minmax").append_prefill(k, v)
    assert cc.kmin is None and cc.kmax is None
    ref = O.build_block_summaries(k.cpu().numpy(), 16, kind="minmax")
    assert np.array_equal(cm.kmax.cpu().numpy(), ref["kmax"])
    assert np.array_equal(cm.kmin.cpu().numpy(), ref["kmin"])
    assert torch.equal(cm.centroid, cc.centroid)
    with pytest.raises(ValueError):
        plan_selection(q, cc, 8, estimator="minmax")
    kq = O.expand_gqa(k.cpu().numpy(), 12)
    vq = O.expand_gqa(v.cpu().numpy(), 12)
    for est, cache in (("centroid", cc), ("minmax", cm)):
        for pol in ("fixed", "adaptive"):
            for ab in (4, 6, 8, 10):
                bt, sl = plan_selection(q, cache, ab, estimator=est, budget_policy=pol,
                                        n_sink_blocks=1, n_local_blocks=2, c_min=1, k_max=256)
                sl = sl.cpu().numpy()
                assert sl.min() - 3 >= 1, f"{est}/{pol}/{ab}: starved"
                if pol == "fixed":
                    assert (sl == max(ab, 4)).all()
            bt, sl = plan_selection(q, cache, 8, estimator=est, budget_policy=pol, n_sink_blocks=1,
                                    n_local_blocks=2, c_min=1, k_max=256)
            torch.cuda.synchronize()
            _, _, mask = O.sparse_attention(q.cpu().numpy(), kq, vq, block_size=16, avg_budget=8, k_min=2,
                                            k_max=256, estimator=est, n_sink_blocks=1, n_local_blocks=2,
                                            c_min=1, budget_policy=pol, return_mask=True)
            bt, sl = bt.cpu().numpy(), sl.cpu().numpy()
            tmask = np.zeros_like(mask)
            for h in range(12):
                tmask[h, bt[h, : sl[h]]] = True
            assert (tmask == mask).mean() > 0.99, f"{est}/{pol}"


def test_minmax_cache_decode_append_and_attention():
    """append_decode refreshes the bounds (equal to a rebuild) and a decode
    step with estimator="minmax" attends over exactly its own selection."""
    from adakv import attention as A
    say("minmax cache append_decode + adakv_decode_attention")
    rng = np.random.RandomState(7)
    Hkv, S, D, G = 4, 2000, 128, 4
    k = torch.from_numpy(rng.standard_normal((Hkv, S + 20, D)).astype(np.float32)).to(torch.bfloat16).to(DEV)
    v = torch.from_numpy(rng.standard_normal((Hkv, S + 20, D)).astype(np.float32)).to(torch.bfloat16).to(DEV)
    q = torch.from_numpy(rng.standard_normal((Hkv * G, D)).astype(np.float32)).to(torch.bfloat16).to(DEV)
    cache = A.AdaKVCache(16, "minmax").append_prefill(k[:, :S], v[:, :S])
    for t in range(20):
        cache.append_decode(k[:, S + t: S + t + 1], v[:, S + t: S + t + 1])
    torch.cuda.synchronize()
    ref = O.build_block_summaries(k.float().cpu().numpy(), 16, kind="minmax")
    assert np.array_equal(cache.kmax.float().cpu().numpy(), ref["kmax"])
    assert np.array_equal(cache.kmin.float().cpu().numpy(), ref["kmin"])
    A.reset_budget_trace()
    out = A.adakv_decode_attention(q, cache, 8, estimator="minmax", budget_policy="fixed")
    bt, sl = A.plan_selection(q, cache, 8, estimator="minmax", budget_policy="fixed")
    trace = A.get_budget_trace()
    A.stop_budget_trace()
    torch.cuda.synchronize()
    assert len(trace) == 2 and trace[0] == trace[1] == 8.0
    o = out.float().cpu().numpy()
    r = O.ref_from_table(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                         bt.cpu().numpy(), sl.cpu().numpy(), 16, G)
    assert np.abs(o - r).max() <= 2e-2
