"""The adaptive_nucleus budget on the GPU, through the C ABI
(adakv/budget.py:38-41, adakv/attention.py:219-221).

The nucleus weight of a head is 1 + the number of its top blocks whose
cumulative softmax mass stays below nucleus_p; the surplus is shared in
proportion to it.  The weight kernel finds that count with a radix search over
exact integer masses; NumPy sums an fp32 running total.  The two agree except
where the exact cumulative mass at the crossing lies within the fp32 running
sum's error of P (gpu_util.nucleus_ambiguous: 1e-6 + K* * 6e-8): such heads
are excluded and counted, and every other head's rounding margin is widened
by what a count moving by one there would shift it.  Elsewhere the GPU is held
to the oracle exactly:

* counts (sel_lens) equal the oracle's allocation on the GPU's own scores, for
  several nucleus masses, temperatures and score distributions;
* the reference's golden nucleus case: mask and counts;
* bf16 / fp16 decode steps (fused kernel): the oracle's selection on the
  GPU's own centroids or minmax bounds, near-ties excluded, and the output of
  fp64 attention over the GPU's own selection;
* the Python API: every (estimator, policy) cell of the reference's factorial
  test runs and agrees with the oracle (tests/test_factorial_selection.py:42-108).
"""
from __future__ import annotations

import numpy as np
import pytest

import cases
import golden_check
from gpu_util import DEV, compare_selection, need_gpu, nucleus_exclusions, say, torch
from oracle import adakv_oracle as O
from test_gpu_fused import _inputs, _params, _run

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    need_gpu()


def _ops():
    from adakv_amd import ops
    return ops


def _budget(ops, p):
    return ops.BudgetParams(avg_budget=p["avg"], k_min=p["kmin"], k_max=p["kmax"],
                            n_sink_blocks=p["sink"], n_local_blocks=p["local"], c_min=p["cmin"],
                            temperature=p["temp"], budget_policy="adaptive_nucleus",
                            nucleus_p=p.get("nucleus_p", 0.9))


@pytest.mark.parametrize("P,T,scale,nb_tokens", [(0.9, 1.0, 1.0, 4096), (0.5, 1.0, 3.0, 4096),
                                                 (0.95, 0.6, 1.0, 2000), (0.9, 1.0, 0.05, 8192),
                                                 (0.75, 1.0, 6.0, 131072 + 48)])
def test_nucleus_counts_match_oracle_on_gpu_scores(P, T, scale, nb_tokens):
    """sel_lens from the plan equal the oracle's nucleus allocation on the
    GPU's own fp32 scores (flat, N(0,1) and peaked heads; 125 to 8195 blocks,
    the last on the 1024-thread x 16 weight kernel)."""
    ops = _ops()
    say(f"nucleus counts P={P} T={T} key scale {scale} S={nb_tokens}")
    rng = np.random.RandomState(int(P * 100) + nb_tokens)
    Hq, Hkv, D, bs = 32, 8, 64, 16
    K = rng.standard_normal((1, Hkv, nb_tokens, D)).astype(np.float32) * np.float32(scale)
    K[:, : Hkv // 2] *= np.float32(2.0)
    q = rng.standard_normal((1, Hq, D)).astype(np.float32)
    k = torch.from_numpy(K).to(DEV)
    qt = torch.from_numpy(q).to(DEV)
    c = ops.centroid_build(k, bs)
    p = dict(avg=12, kmin=2, kmax=256, sink=1, local=4, cmin=1, temp=T, nucleus_p=P)
    sc = ops.block_scores(qt, c, bs, seq_len=nb_tokens)
    table, lens = ops.plan(qt, c, bs, _budget(ops, p), seq_len=nb_tokens)
    torch.cuda.synchronize()
    nb = ops.n_blocks(nb_tokens, bs)
    scores = sc[0, :, :nb].cpu().numpy()
    lo, _, target, _ = O.budget_bounds(nb, p["avg"], p["kmin"], p["kmax"], p["sink"], p["local"], p["cmin"])
    amb, margin = nucleus_exclusions(scores, lo, target, T, P)
    k_or = O.allocate_budget(scores, p["avg"], min(p["kmin"], nb), min(p["kmax"], nb), temperature=T,
                             policy="adaptive_nucleus", nucleus_p=P,
                             floor=min(p["sink"], nb) + min(p["local"], nb) + p["cmin"])
    w = O.budget_weights(scores, "adaptive_nucleus", T, P)
    say(f"  nucleus weights {int(w.min())} .. {int(w.max())}, counts {int(k_or.min())} .. {int(k_or.max())}, "
        f"{int(amb.sum())} knife-edge heads")
    excl = compare_selection(scores, table[0].cpu().numpy(), lens[0].cpu().numpy(), k_oracle=k_or,
                             w_oracle=w, lo=lo, target=target, sink=p["sink"], local=p["local"],
                             cmin=p["cmin"], policy="adaptive_nucleus", exclude=amb, half_margin=margin)
    say(f"  {excl} heads excluded")


@pytest.mark.parametrize("P", [0.95])
def test_nucleus_crossing_in_the_tail_bin(P):
    """One dominant block per KV head and 8191 blocks more than 255/16 octaves
    of probability below it: for most heads the crossing of P falls in the
    radix search's last (tail) bin, so the weight kernel takes its four extra
    passes over all 31 bits of the distance.  Centroids are set directly
    (score = q[0] * c[0]).  Counts are held to the oracle's on the GPU's own
    scores wherever NumPy's fp32 running sum fixes them; a tail crossing sums
    about 10^3 terms of 1e-5, inside that sum's error, so every head's count
    is also held to the fp64 cumulative sum of the same fp32 probabilities,
    which the kernel's exact integer masses reproduce (with at least 4 heads
    crossing in the tail among those checked)."""
    ops = _ops()
    Hq, Hkv, D, bs, S = 32, 8, 64, 16, 131072
    G = Hq // Hkv
    nb = S // bs
    say(f"nucleus tail crossing P={P}, {nb} blocks")
    rng = np.random.RandomState(int(P * 1000))
    C = np.zeros((1, Hkv, nb, D), np.float32)
    for g in range(Hkv):
        C[0, g, :, 0] = (-11.3 - 0.05 * g + rng.uniform(-0.15, 0.15, nb)).astype(np.float32)
        C[0, g, 100 + 7 * g, 0] = 0.0
    q = np.zeros((1, Hq, D), np.float32)
    for h in range(Hq):
        q[0, h, 0] = np.float32(1.0 + 0.02 * (h % G))
    c = torch.from_numpy(C).to(DEV)
    qt = torch.from_numpy(q).to(DEV)
    p = dict(avg=12, kmin=2, kmax=256, sink=1, local=4, cmin=1, temp=1.0, nucleus_p=P)
    sc = ops.block_scores(qt, c, bs, seq_len=S)
    table, lens = ops.plan(qt, c, bs, _budget(ops, p), seq_len=S)
    torch.cuda.synchronize()
    scores = sc[0, :, :nb].cpu().numpy()
    # the branch is reached: the crossing block lies more than 255/16 octaves below the maximum
    z = scores.astype(np.float64) - scores.max(axis=1, keepdims=True)
    pr = np.sort(np.exp(z) / np.exp(z).sum(axis=1, keepdims=True), axis=1)[:, ::-1]
    kstar = (np.cumsum(pr, axis=1) < P).sum(axis=1)
    deep = np.log2(pr[np.arange(Hq), kstar] / pr[:, 0]) < -255.0 / 16
    say(f"  {int(deep.sum())}/{Hq} heads cross P in the tail bin")
    assert deep.sum() >= 8
    lo, _, target, _ = O.budget_bounds(nb, p["avg"], p["kmin"], p["kmax"], p["sink"], p["local"], p["cmin"])
    amb, margin = nucleus_exclusions(scores, lo, target, 1.0, P)
    k_or = O.allocate_budget(scores, p["avg"], min(p["kmin"], nb), min(p["kmax"], nb), temperature=1.0,
                             policy="adaptive_nucleus", nucleus_p=P,
                             floor=min(p["sink"], nb) + min(p["local"], nb) + p["cmin"])
    w = O.budget_weights(scores, "adaptive_nucleus", 1.0, P)
    say(f"  nucleus weights {int(w.min())} .. {int(w.max())}, {int(amb.sum())} knife-edge heads")
    # the 8191 low scores lie within 0.4 of each other, so most heads' selections
    # end on a score near-tie; what this case pins is the counts, compared on
    # every head whose budget is not at a rounding knife-edge
    excl = compare_selection(scores, table[0].cpu().numpy(), lens[0].cpu().numpy(), k_oracle=k_or,
                             w_oracle=w, lo=lo, target=target, sink=p["sink"], local=p["local"],
                             cmin=p["cmin"], policy="adaptive_nucleus", exclude=amb, half_margin=margin,
                             max_excluded=1.0)
    counted = ~(O.budget_near_half(w, lo, target, margin=margin) | amb)
    say(f"  counts compared on {int(counted.sum())} heads ({int((counted & deep).sum())} crossing in the tail), "
        f"{excl} heads excluded from the selection comparison")
    assert counted.sum() >= 8
    k = lens[0].cpu().numpy()
    floor = min(p["sink"], nb) + min(p["local"], nb) + p["cmin"]
    assert np.all(k >= max(lo, floor)) and np.all(k <= max(min(p["kmax"], nb), floor))
    # The tail branch pinned against an fp64 cumulative sum.  The weight
    # kernel adds the probabilities' masses exactly, so its K* is the fp64
    # count of the same fp32 probabilities wherever the crossing is farther
    # from P than their own last-ulp differences (2e-7 of the whole mass);
    # NumPy's fp32 running sum is no reference there (10^3 terms of 1e-5).
    z = scores.astype(np.float32)
    p32 = np.exp(z - z.max(axis=1, keepdims=True))
    p32 /= p32.sum(axis=1, keepdims=True)
    c64 = np.cumsum(np.sort(p32.astype(np.float64), axis=1)[:, ::-1], axis=1)
    P32 = float(np.float32(P))
    w64 = (c64 < P32).sum(axis=1).astype(np.float64) + 1.0
    edge = np.zeros(Hq, bool)
    for h in range(Hq):
        kk = int(w64[h])
        for j in (kk - 2, kk - 1):
            if 0 <= j < nb and abs(c64[h, j] - P32) <= 2e-7:
                edge[h] = True
    extra64 = O.budget_extra(w64, lo, target)
    margin64 = max(1e-3, 2.0 * float(edge.sum()) * float(extra64.max()) / float(w64.sum()) + 1e-4)
    hi = min(p["kmax"], nb)
    k64 = np.minimum(np.maximum(np.clip(np.round(lo + extra64), lo, hi).astype(np.int64), floor), nb)
    checked = ~(edge | O.budget_near_half(w64, lo, target, margin=margin64))
    say(f"  fp64 counts: {int(checked.sum())} heads checked, {int((checked & deep).sum())} crossing in the tail, "
        f"{int(edge.sum())} at the edge")
    bad = [(h, int(k[h]), int(k64[h])) for h in range(Hq) if checked[h] and k[h] != k64[h]]
    assert not bad, f"counts differ from the fp64 nucleus count on heads {bad[:8]}"
    assert (checked & deep).sum() >= 4, "fewer than 4 tail-crossing heads had their counts checked"


def test_nucleus_plan_matches_reference_golden():
    """fp32 path vs the reference's own mask and counts (golden nucleus case)."""
    ops = _ops()
    name = "nucleus"
    say(f"nucleus plan golden {name}")
    p = cases.params(name)
    q, Kkv, _ = cases.make_inputs(name)
    g = golden_check.load(name)
    bs = p["bs"]
    k = torch.from_numpy(Kkv).to(DEV).unsqueeze(0)
    c = ops.centroid_build(k, bs)
    qt = torch.from_numpy(q).to(DEV).unsqueeze(0)
    table, lens = ops.plan(qt, c, bs, _budget(ops, p), seq_len=Kkv.shape[1])
    torch.cuda.synchronize()
    nb = g["scores"].shape[1]
    table, lens = table[0].cpu().numpy(), lens[0].cpu().numpy()
    lo, _, target, _ = O.budget_bounds(nb, p["avg"], p["kmin"], p["kmax"], p["sink"], p["local"], p["cmin"])
    amb, margin = nucleus_exclusions(g["scores"], lo, target, p["temp"], 0.9)
    w = O.budget_weights(g["scores"], "adaptive_nucleus", p["temp"], 0.9)
    excl = compare_selection(g["scores"], table, lens, k_oracle=g["k"], w_oracle=w, lo=lo, target=target,
                             sink=p["sink"], local=p["local"], cmin=p["cmin"], policy="adaptive_nucleus",
                             exclude=amb, half_margin=margin)
    say(f"  {excl} heads excluded")
    if excl == 0:
        gm = np.zeros_like(g["mask"])
        for h in range(table.shape[0]):
            gm[h, table[h, : lens[h]]] = True
        assert np.array_equal(gm, g["mask"])
        assert np.array_equal(lens, g["counts"])


@pytest.mark.parametrize("name", ["nucleus", "cfg1_seed0", "peaked_mixed", "partial_tail", "gqa6_kmax256",
                                  "bs32", "planted", "tiny_overlap"])
def test_nucleus_fused_bf16_golden_inputs(name):
    p = cases.params(name)
    p.update(policy="adaptive_nucleus", est="centroid")
    say(f"nucleus fused bf16 {name}")
    q, K, V = cases.make_inputs(name)
    _run(q[None], K[None], V[None], p, p["bs"], torch.bfloat16)


def test_nucleus_fused_fp16_minmax():
    """The budget-only cell's nucleus variant: minmax bounds scored, nucleus budget."""
    p = cases.params("nucleus")
    p.update(est="minmax")
    say("nucleus fused fp16 with minmax bounds")
    q, K, V = cases.make_inputs("nucleus")
    _run(q[None], K[None], V[None], p, p["bs"], torch.float16)


@pytest.mark.parametrize("Hq,Hkv,D,P", [(64, 8, 64, 0.9), (40, 5, 128, 0.8), (16, 4, 32, 0.5)])
def test_nucleus_fused_many_heads(Hq, Hkv, D, P):
    say(f"nucleus fused Hq={Hq} Hkv={Hkv} D={D} P={P}")
    q, K, V = _inputs(41, 1, Hq, Hkv, 4096, D)
    _run(q, K, V, _params(avg=10, policy="adaptive_nucleus", nucleus_p=P), 16, torch.bfloat16)


def test_nucleus_fused_append_and_ragged():
    say("nucleus fused append 40 tokens; ragged batch [0, 1, 777, 4096]")
    q, K, V = _inputs(42, 1, 32, 8, 4096 + 7, 128)
    _run(q, K, V, _params(avg=8, policy="adaptive_nucleus"), 16, torch.bfloat16, append_new=40,
         corrupt_tail=40)
    q, K, V = _inputs(43, 4, 16, 4, 4096, 128)
    _run(q, K, V, _params(avg=8, policy="adaptive_nucleus", temp=0.7), 16, torch.bfloat16,
         seq_lens=[0, 1, 777, 4096])


def test_nucleus_fused_equals_plan_then_decode():
    """The fused step (score, weight, selection + decode kernels) and the plan
    + table-driven decode agree on the counts and selections."""
    ops = _ops()
    say("nucleus fused vs plan + sparse decode")
    q, K, V = _inputs(44, 1, 32, 8, 8192, 128)
    qd, kd, vd = (torch.from_numpy(x).to(torch.bfloat16).to(DEV) for x in (q, K, V))
    c = ops.centroid_build(kd, 16)
    budget = ops.BudgetParams(avg_budget=8, budget_policy="adaptive_nucleus")
    out_f, table_f, lens_f = ops.decode_fused(qd, kd, vd, c, 16, budget, return_selection=True)
    table_p, lens_p = ops.plan(qd, c, 16, budget, seq_len=8192)
    out_p = ops.sparse_decode(qd, kd, vd, table_p, lens_p, 16)
    torch.cuda.synchronize()
    assert torch.equal(lens_f, lens_p)
    lf, tf_, tp = lens_f[0].cpu().numpy(), table_f[0].cpu().numpy(), table_p[0].cpu().numpy()
    same = [h for h in range(32) if set(tf_[h, :lf[h]]) == set(tp[h, :lf[h]])]
    assert len(same) >= 28
    assert (out_f[0, same].float() - out_p[0, same].float()).abs().max().item() <= 1e-2


def test_all_six_factorial_cells_match_the_oracle():
    """tests/test_factorial_selection.py:42-108 with every policy built:
    all cells run, keep >= c_min content blocks, fixed honours its budget,
    adaptive policies land near the target mean, masks agree with the oracle."""
    from adakv.attention import AdaKVCache, plan_selection
    say("factorial cells incl. adaptive_nucleus")
    rng = np.random.RandomState(0)
    k = torch.from_numpy(rng.standard_normal((2, 320, 64)).astype(np.float32)).to(DEV)
    v = torch.from_numpy(rng.standard_normal((2, 320, 64)).astype(np.float32)).to(DEV)
    q = torch.from_numpy(rng.standard_normal((12, 64)).astype(np.float32)).to(DEV)
    caches = {"centroid": AdaKVCache(16, "centroid").append_prefill(k, v),
              "minmax": AdaKVCache(16, "minmax").append_prefill(k, v)}
    kq, vq, qn = O.expand_gqa(k.cpu().numpy(), 12), O.expand_gqa(v.cpu().numpy(), 12), q.cpu().numpy()
    common = dict(n_sink_blocks=1, n_local_blocks=2, c_min=1, k_max=256)
    for est, cache in caches.items():
        for pol in ("fixed", "adaptive", "adaptive_nucleus"):
            for ab in (4, 6, 8):
                _, sl = plan_selection(q, cache, ab, estimator=est, budget_policy=pol, **common)
                assert int(sl.min()) - 3 >= 1, f"{est}/{pol}/{ab}: starved"
            _, sl = plan_selection(q, cache, 8, estimator=est, budget_policy=pol, **common)
            m = float(sl.float().mean())
            assert 4 <= m <= 10, f"{est}/{pol}: realised mean {m}"
            bt, sl = plan_selection(q, cache, 8, estimator=est, budget_policy=pol, **common)
            torch.cuda.synchronize()
            _, _, mask = O.sparse_attention(qn, kq, vq, block_size=16, avg_budget=8, k_min=2, k_max=256,
                                            estimator=est, n_sink_blocks=1, n_local_blocks=2, c_min=1,
                                            budget_policy=pol, return_mask=True)
            bt, sl = bt.cpu().numpy(), sl.cpu().numpy()
            tmask = np.zeros_like(mask)
            for h in range(12):
                tmask[h, bt[h, : sl[h]]] = True
            assert (tmask == mask).mean() > 0.99, f"{est}/{pol}"
