"""HIP path vs the oracle: centroids, plan (scores + budget + selection),
sparse decode, fused step, dense decode.  Every call goes through the C ABI of
libadakv_amd.so (via adakv_amd.ops)."""
from __future__ import annotations

import math

import numpy as np
import pytest

import cases
import golden_check
from gpu_util import (BF16_ATOL, DEV, REL_L2, compare_selection, need_gpu, rel_l2, say, to_np,
                      torch)
from oracle import adakv_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    need_gpu()


def _ops():
    from adakv_amd import ops
    return ops


def _bf16_round(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


# ------------------------------------------------------------------ centroids
@pytest.mark.parametrize("S,D,bs", [(4001, 64, 16), (4096, 128, 16), (1000, 32, 32), (300, 256, 16),
                                    (37, 128, 5)])
def test_centroid_build_fp32_bit_exact(S, D, bs):
    ops = _ops()
    say(f"centroid fp32 S={S} D={D} bs={bs}")
    rng = np.random.RandomState(S + D)
    K = rng.standard_normal((3, S, D)).astype(np.float32)
    c = ops.centroid_build(torch.from_numpy(K).to(DEV).unsqueeze(0), bs)
    torch.cuda.synchronize()
    ref = O.build_block_summaries(K, bs)["centroid"]
    got = c[0].cpu().numpy()
    assert got.dtype == np.float32 and np.array_equal(got[:, : ref.shape[1]], ref)


def test_centroid_build_bf16_keys():
    ops = _ops()
    say("centroid bf16 keys -> bf16 / fp32 centroids")
    rng = np.random.RandomState(3)
    Kb = torch.from_numpy(rng.standard_normal((1, 8, 2000, 128)).astype(np.float32)).to(torch.bfloat16)
    ref = O.build_block_summaries(Kb[0].float().numpy(), 16)["centroid"]
    c32 = ops.centroid_build(Kb.to(DEV), 16, centroid_dtype=torch.float32)
    c16 = ops.centroid_build(Kb.to(DEV), 16)
    torch.cuda.synchronize()
    assert c16.dtype == torch.bfloat16
    assert np.array_equal(c32[0].cpu().numpy(), ref)
    assert np.array_equal(c16[0].float().cpu().numpy(), _bf16_round(ref))


def test_centroid_append_equals_rebuild():
    ops = _ops()
    say("centroid append vs rebuild")
    rng = np.random.RandomState(4)
    Hkv, S0, D, bs, steps = 4, 100, 64, 16, 50
    K = torch.from_numpy(rng.standard_normal((1, Hkv, S0 + steps, D)).astype(np.float32)).to(DEV)
    cap = ops.n_blocks(S0 + steps, bs) + 3
    c = ops.centroid_build(K[:, :, :S0], bs, max_blocks=cap)
    for t in range(steps):
        ops.centroid_append(K[:, :, : S0 + t + 1], c, bs, n_new=1)
    c2 = ops.centroid_build(K, bs, max_blocks=cap)
    ops.centroid_append(K, c2, bs, n_new=37)      # multi-token append spanning blocks
    torch.cuda.synchronize()
    full = O.build_block_summaries(K[0].cpu().numpy(), bs)["centroid"]
    nb = full.shape[1]
    assert np.array_equal(c[0, :, :nb].cpu().numpy(), full)
    assert np.array_equal(c2[0, :, :nb].cpu().numpy(), full)


# ------------------------------------------------------------------ planning
PLAN_CASES = [n for n in sorted(cases.CASES)
              if cases.params(n)["est"] == "centroid" and cases.params(n)["policy"] != "adaptive_nucleus"
              and cases.params(n)["temp"] == 1.0]


def _plan_case(name, centroid_dtype=torch.float32):
    ops = _ops()
    p = cases.params(name)
    q, Kkv, Vkv = cases.make_inputs(name)
    bs = p["bs"]
    budget = ops.BudgetParams(avg_budget=p["avg"], k_min=p["kmin"], k_max=p["kmax"],
                              n_sink_blocks=p["sink"], n_local_blocks=p["local"], c_min=p["cmin"],
                              budget_policy=p["policy"])
    k = torch.from_numpy(Kkv).to(DEV).unsqueeze(0)
    c = ops.centroid_build(k, bs, centroid_dtype=centroid_dtype)
    qt = torch.from_numpy(q).to(DEV).unsqueeze(0)
    table, lens = ops.plan(qt, c, bs, budget, seq_len=Kkv.shape[1])
    torch.cuda.synchronize()
    return p, q, Kkv, Vkv, c, table[0].cpu().numpy(), lens[0].cpu().numpy()


@pytest.mark.parametrize("name", PLAN_CASES)
def test_plan_matches_reference_golden(name):
    """GPU selection vs the reference's own mask / counts (golden fixture)."""
    say(f"plan golden {name}")
    p, q, Kkv, Vkv, c, table, lens = _plan_case(name)
    g = golden_check.load(name)
    nb = g["scores"].shape[1]
    lo, hi, target, _ = O.budget_bounds(nb, p["avg"], p["kmin"], p["kmax"], p["sink"], p["local"],
                                        p["cmin"])
    k_or = g["k"]
    w = g.get("w", np.ones(q.shape[0]))
    excl = compare_selection(g["scores"], table, lens, k_oracle=k_or, w_oracle=w, lo=lo,
                             target=target, sink=p["sink"], local=p["local"], cmin=p["cmin"],
                             policy=p["policy"])
    # where nothing was excluded, the GPU mask is the reference's mask exactly
    if excl == 0:
        gm = np.zeros_like(g["mask"])
        for h in range(table.shape[0]):
            gm[h, table[h, : lens[h]]] = True
        assert np.array_equal(gm, g["mask"])
        assert np.array_equal(lens, g["counts"])


@pytest.mark.parametrize("name", PLAN_CASES)
def test_centroid_block_scores_match_reference_golden(name):
    """adakv_block_scores on fp32 centroids (the VALU scan) against the
    reference's own fp32 scores of the golden fixture, within the fixture's
    score tolerance (2e-6 of the largest magnitude: NumPy's einsum sums in
    another order)."""
    ops = _ops()
    say(f"centroid block scores golden {name}")
    p = cases.params(name)
    q, Kkv, _ = cases.make_inputs(name)
    g = golden_check.load(name)
    k = torch.from_numpy(Kkv).to(DEV).unsqueeze(0)
    c = ops.centroid_build(k, p["bs"])
    s = ops.block_scores(torch.from_numpy(q).to(DEV).unsqueeze(0), c, p["bs"], seq_len=Kkv.shape[1])
    torch.cuda.synchronize()
    nb = g["scores"].shape[1]
    got = s[0, :, :nb].cpu().numpy()
    scale = float(np.abs(g["scores"]).max()) or 1.0
    err = float(np.abs(got - g["scores"]).max())
    say(f"  max |score diff| {err:.2e} (scale {scale:.2e})")
    assert err <= golden_check.SCORE_RTOL * scale


def test_plan_bf16_centroids_match_oracle_on_same_centroids():
    """bf16 centroids: the oracle budget + selection run on the GPU's stored centroids."""
    ops = _ops()
    say("plan bf16 centroids cfg1")
    p, q, Kkv, Vkv, c, table, lens = _plan_case("cfg1_seed0", centroid_dtype=torch.bfloat16)
    nb = ops.n_blocks(Kkv.shape[1], p["bs"])
    cent = O.expand_gqa(c[0, :, :nb].float().cpu().numpy(), q.shape[0])
    scores = O.block_scores(q, {"kind": "centroid", "centroid": cent})
    lo, hi, target, _ = O.budget_bounds(nb, p["avg"], p["kmin"], p["kmax"], p["sink"], p["local"],
                                        p["cmin"])
    k = O.allocate_budget(scores, p["avg"], min(p["kmin"], nb), min(p["kmax"], nb),
                          floor=min(p["sink"], nb) + min(p["local"], nb) + p["cmin"])
    w = O.budget_weights(scores)
    compare_selection(scores, table, lens, k_oracle=k, w_oracle=w, lo=lo, target=target,
                      sink=p["sink"], local=p["local"], cmin=p["cmin"], policy=p["policy"])


def test_plan_temperature_case():
    say("plan temperature 0.5")
    p, q, Kkv, Vkv, c, table, lens = _plan_case("temp_sink_local")
    ops = _ops()
    g = golden_check.load("temp_sink_local")
    nb = g["scores"].shape[1]
    lo, hi, target, _ = O.budget_bounds(nb, p["avg"], p["kmin"], p["kmax"], p["sink"], p["local"],
                                        p["cmin"])
    # the fixture for this case was recorded with temperature 0.5 (k_temp, w)
    budget = ops.BudgetParams(avg_budget=p["avg"], k_min=p["kmin"], k_max=p["kmax"],
                              n_sink_blocks=p["sink"], n_local_blocks=p["local"], c_min=p["cmin"],
                              temperature=p["temp"])
    table_t, lens_t = ops.plan(torch.from_numpy(q).to(DEV).unsqueeze(0), c, p["bs"], budget,
                               seq_len=Kkv.shape[1])
    torch.cuda.synchronize()
    compare_selection(g["scores"], table_t[0].cpu().numpy(), lens_t[0].cpu().numpy(),
                      k_oracle=g["k_temp"], w_oracle=g["w"], lo=lo, target=target, sink=p["sink"],
                      local=p["local"], cmin=p["cmin"], policy="adaptive")


def test_plan_ragged_batch_matches_per_sequence_oracle():
    ops = _ops()
    say("plan ragged batch B=4")
    rng = np.random.RandomState(21)
    B, Hq, Hkv, D, bs = 4, 16, 4, 64, 16
    lens_tok = np.array([1000, 37, 4096, 2500], np.int32)
    S = int(lens_tok.max())
    K = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    K[:2] *= 3.0
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    kt = torch.from_numpy(K).to(DEV)
    sl = torch.from_numpy(lens_tok).to(DEV)
    c = ops.centroid_build(kt, bs, seq_lens=sl)
    budget = ops.BudgetParams(avg_budget=12)
    table, lens = ops.plan(torch.from_numpy(q).to(DEV), c, bs, budget, seq_len=S, seq_lens=sl)
    torch.cuda.synchronize()
    table, lens = table.cpu().numpy(), lens.cpu().numpy()
    for b in range(B):
        Sb = int(lens_tok[b])
        Kb = O.expand_gqa(K[b, :, :Sb], Hq)
        summ = O.build_block_summaries(Kb, bs)
        scores = O.block_scores(q[b], summ)
        nb = summ["n_blocks"]
        lo, hi, target, _ = O.budget_bounds(nb, 12, 2, 64, 1, 4, 1)
        k = O.allocate_budget(scores, 12, min(2, nb), min(64, nb), floor=min(1, nb) + min(4, nb) + 1)
        w = O.budget_weights(scores) if nb > 1 else np.ones(Hq)
        compare_selection(scores, table[b], lens[b], k_oracle=k, w_oracle=w, lo=lo, target=target,
                          sink=1, local=4, cmin=1, policy="adaptive")


# ------------------------------------------------------------------ decoding
def _random_table(rng, Hq, nb, width, lens):
    t = np.full((Hq, width), -1, np.int32)
    for h in range(Hq):
        n = int(lens[h])
        t[h, :n] = rng.choice(nb, size=n, replace=n > nb)
    return t


@pytest.mark.parametrize("Hkv,group,S,D,bs,dt", [
    (8, 4, 4096, 128, 16, torch.float16),      # tests/test_kernel_parity.py:46
    (4, 1, 8192, 64, 32, torch.float16),
    (8, 4, 4096, 128, 16, torch.bfloat16),
    (2, 8, 1000, 128, 16, torch.bfloat16),      # GQA 8, partial tail block
    (2, 3, 777, 32, 8, torch.float32),
    (2, 3, 777, 32, 8, torch.bfloat16),         # blocks shorter than a 16-token tile
    (2, 4, 1500, 64, 24, torch.float16),        # blocks of 1.5 tiles, padded q-heads
    (2, 2, 600, 256, 16, torch.bfloat16),
    (8, 16, 2048, 128, 16, torch.bfloat16),     # GQA 16: 128 q / 8 KV heads
    (1, 16, 700, 256, 16, torch.float32),       # GQA 16, head_dim 256, vector-unit decode
    (2, 16, 900, 64, 24, torch.float16),
])
def test_sparse_decode_matches_same_selection_reference(Hkv, group, S, D, bs, dt):
    ops = _ops()
    say(f"sparse decode Hkv={Hkv} G={group} S={S} D={D} bs={bs} {dt}")
    rng = np.random.RandomState(S + D + bs)
    Hq = Hkv * group
    nb = ops.n_blocks(S, bs)
    q = torch.randn(1, Hq, D, generator=torch.Generator().manual_seed(0)).to(dt)
    k = (torch.randn(1, Hkv, S, D, generator=torch.Generator().manual_seed(1)) * 0.1).to(dt)
    v = torch.randn(1, Hkv, S, D, generator=torch.Generator().manual_seed(2)).to(dt)
    width = 24
    lens = rng.randint(1, width + 1, size=Hq).astype(np.int32)
    table = _random_table(rng, Hq, nb, width, lens)
    table[0, 0] = nb + 5               # out-of-range id: ignored
    if lens[1] >= 2:
        table[1, 1] = table[1, 0]      # duplicate: counted once
    out = ops.sparse_decode(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(table).to(DEV)[None],
                            torch.from_numpy(lens).to(DEV)[None], bs)
    torch.cuda.synchronize()
    ref = O.ref_from_table(to_np(q[0]), to_np(k[0]), to_np(v[0]), table, lens, bs, group)
    got = to_np(out[0])
    ok = np.isfinite(ref).all(axis=1)
    assert ok.sum() >= Hq - 1
    err = np.abs(got[ok] - ref[ok]).max()
    assert rel_l2(got[ok], ref[ok]) < REL_L2 and err <= BF16_ATOL, (rel_l2(got[ok], ref[ok]), err)
    if dt == torch.float32:
        assert err <= 1e-4


def test_sparse_decode_empty_rows_give_nan_like_reference():
    ops = _ops()
    say("sparse decode empty rows")
    q = torch.randn(1, 4, 64).to(DEV)
    k = torch.randn(1, 2, 64, 64).to(DEV)
    table = torch.full((1, 4, 3), -1, dtype=torch.int32, device=DEV)
    lens = torch.tensor([[0, 3, 1, 0]], dtype=torch.int32, device=DEV)
    table[0, 2, 0] = 1
    out = ops.sparse_decode(q, k, k, table, lens, 16)
    torch.cuda.synchronize()
    o = out[0].cpu().numpy()
    assert np.isnan(o[0]).all() and np.isnan(o[1]).all() and np.isnan(o[3]).all()
    assert np.isfinite(o[2]).all()


@pytest.mark.parametrize("name", ["cfg1_seed0", "cfg1_seed3_avg32", "partial_tail", "gqa6_kmax256",
                                  "bs32", "tiny_overlap", "single_block", "planted"])
def test_fused_step_matches_oracle_output(name):
    """plan + decode in one C call vs the reference's sparse_attention output
    (golden), on every head whose selection matched."""
    ops = _ops()
    say(f"fused golden {name}")
    p = cases.params(name)
    q, Kkv, Vkv = cases.make_inputs(name)
    g = golden_check.load(name)
    bs = p["bs"]
    budget = ops.BudgetParams(avg_budget=p["avg"], k_min=p["kmin"], k_max=p["kmax"],
                              n_sink_blocks=p["sink"], n_local_blocks=p["local"], c_min=p["cmin"],
                              budget_policy=p["policy"])
    k = torch.from_numpy(Kkv).to(DEV).unsqueeze(0)
    v = torch.from_numpy(Vkv).to(DEV).unsqueeze(0)
    c = ops.centroid_build(k, bs)
    out, table, lens = ops.decode_fused(torch.from_numpy(q).to(DEV).unsqueeze(0), k, v, c, bs, budget,
                                        return_selection=True)
    torch.cuda.synchronize()
    table, lens, got = table[0].cpu().numpy(), lens[0].cpu().numpy(), out[0].cpu().numpy()
    # the fused kernel's own counts and selection, held to the same rule as the
    # plan's: the reference's counts and masks on every head that is not a
    # near-half count or a near-tie at the boundary (excluded and counted)
    nb = g["scores"].shape[1]
    lo, hi, target, _ = O.budget_bounds(nb, p["avg"], p["kmin"], p["kmax"], p["sink"], p["local"],
                                        p["cmin"])
    excl = compare_selection(g["scores"], table, lens, k_oracle=g["k"] if "k" in g else g["counts"],
                             w_oracle=g.get("w", np.ones(q.shape[0])),
                             lo=lo, target=target, sink=p["sink"], local=p["local"], cmin=p["cmin"],
                             policy=p["policy"])
    say(f"  selection parity: {q.shape[0] - excl}/{q.shape[0]} heads compared, {excl} excluded as near-ties")
    same = np.zeros(q.shape[0], bool)
    for h in range(q.shape[0]):
        same[h] = set(table[h, : lens[h]].tolist()) == set(np.flatnonzero(g["mask"][h]).tolist())
    assert same.sum() >= q.shape[0] - excl
    assert np.abs(got[same] - g["out"][same]).max() <= 2e-4
    # every head, matched or not, equals attention over its own selection
    ref = O.ref_from_table(q, Kkv, Vkv, table, lens, bs, q.shape[0] // Kkv.shape[0])
    assert np.abs(got - ref).max() <= 2e-4


@pytest.mark.parametrize("S,dt,G", [(4096, torch.float32, 4), (20000, torch.bfloat16, 4), (777, torch.float16, 4),
                                    (5000, torch.bfloat16, 16), (1000, torch.float32, 16)])
def test_dense_decode_matches_fp64_dense(S, dt, G):
    ops = _ops()
    say(f"dense decode S={S} {dt} group {G}")
    Hkv, D = 8, 128
    q = torch.randn(1, Hkv * G, D).to(dt)
    k = torch.randn(1, Hkv, S, D).to(dt)
    v = torch.randn(1, Hkv, S, D).to(dt)
    out = ops.dense_decode(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    ref = O.dense_attention(to_np(q[0]).astype(np.float64), O.expand_gqa(to_np(k[0]), Hkv * G),
                            O.expand_gqa(to_np(v[0]), Hkv * G))
    got = to_np(out[0])
    tol = 1e-4 if dt == torch.float32 else BF16_ATOL
    assert np.abs(got - ref).max() <= tol and rel_l2(got, ref) < REL_L2


def test_full_budget_equals_dense():
    """tests/test_runtime_cpu.py:47-59 on the GPU: every block selected == dense."""
    ops = _ops()
    say("full budget == dense")
    Hkv, G, S, D, bs = 4, 2, 256, 64, 16
    nb = S // bs
    q = torch.randn(1, Hkv * G, D, device=DEV)
    k = torch.randn(1, Hkv, S, D, device=DEV) * 0.1
    v = torch.randn(1, Hkv, S, D, device=DEV)
    c = ops.centroid_build(k, bs)
    out = ops.decode_fused(q, k, v, c, bs, ops.BudgetParams(avg_budget=nb, k_min=nb, k_max=nb))
    dense = ops.dense_decode(q, k, v)
    torch.cuda.synchronize()
    assert rel_l2(out.cpu().numpy(), dense.cpu().numpy()) < 1e-5
