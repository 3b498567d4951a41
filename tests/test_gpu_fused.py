"""The fused budget + selection + decode path for bf16 / fp16 K/V, through the C ABI.

The golden inputs are fp32; here q, K and V are rounded to bf16 (or fp16) and
the centroids are built on the GPU in that type, so every check runs on what
the GPU actually used:

* selection: the oracle's budget (adakv/budget.py:45-86) and selection
  (adakv/selector.py:18-60) on the GPU's own centroids, read back after the
  step (appended blocks carry their recomputed centroids), compared
  bit-exactly with near-ties excluded and counted;
* output: fp64 attention over the GPU's own selection
  (tests/test_kernel_parity.py:25-43), within the bf16 tolerance.

The cases cover the kernel's branches: adaptive and fixed budgets, a
temperature, q-head counts above 32 (several merge passes), head_dim 32 / 64 /
128, block sizes 16 / 24 / 32 (a non-power-of-two division, two 16-token tiles
per block), wide tables (k_max 256), k_min above the floor and k_max below it,
single-block and overlapping sink/local sequences, an append of several rows,
and a ragged batch holding an empty and a one-token sequence.
"""
from __future__ import annotations

import numpy as np
import pytest

import cases
from gpu_util import BF16_ATOL, DEV, REL_L2, compare_selection, need_gpu, nucleus_exclusions, rel_l2, say, torch
from oracle import adakv_oracle as O

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
                            temperature=p["temp"], budget_policy=p["policy"],
                            nucleus_p=p.get("nucleus_p", 0.9))


def _rounded(x: np.ndarray, dt) -> np.ndarray:
    return torch.from_numpy(x).to(dt).float().numpy()


def summary_of(c: np.ndarray, Hq: int, est: str) -> dict:
    """The oracle's summary dict from GPU summaries [Hkv, nb, D] (centroid) or
    [Hkv, nb, 2D] (minmax rows [max | min]), expanded to the q-heads."""
    c = O.expand_gqa(c.astype(np.float32), Hq)
    if est == "minmax":
        D = c.shape[-1] // 2
        return {"kind": "minmax", "kmax": np.ascontiguousarray(c[..., :D]),
                "kmin": np.ascontiguousarray(c[..., D:])}
    return {"kind": "centroid", "centroid": c}


def _check_sequence(q, K, V, c, table, lens, out, p, bs, tag):
    """One sequence: q [Hq, D], K/V [Hkv, S, D] (the rounded values), c the
    GPU summaries [Hkv, nb, D or 2D]; table [Hq, T], lens [Hq], out [Hq, D]."""
    Hq, Hkv = q.shape[0], K.shape[0]
    nb = c.shape[1]
    scores = O.block_scores(q, summary_of(c, Hq, p.get("est", "centroid")))
    lo, _, target, _ = O.budget_bounds(nb, p["avg"], p["kmin"], p["kmax"], p["sink"], p["local"], p["cmin"])
    floor = min(p["sink"], nb) + min(p["local"], nb) + p["cmin"]
    P = p.get("nucleus_p", 0.9)
    k = O.allocate_budget(scores, p["avg"], min(p["kmin"], nb), min(p["kmax"], nb),
                          temperature=p["temp"], policy=p["policy"], nucleus_p=P, floor=floor)
    w = O.budget_weights(scores, "adaptive_nucleus" if p["policy"] == "adaptive_nucleus" else "adaptive",
                         p["temp"], P)
    amb, margin = None, 1e-3
    if p["policy"] == "adaptive_nucleus" and nb > 1:
        # nucleus counts on a rounding knife-edge: excluded, and the others'
        # rounding margin widened by what they would move
        amb, margin = nucleus_exclusions(scores, lo, target, p["temp"], P)
    excl = compare_selection(scores, table, lens, k_oracle=k, w_oracle=w, lo=lo, target=target,
                             sink=p["sink"], local=p["local"], cmin=p["cmin"], policy=p["policy"],
                             exclude=amb, half_margin=margin)
    ref = O.ref_from_table(q, K, V, table, lens, bs, Hq // Hkv)
    err = float(np.abs(out - ref).max())
    r = rel_l2(out, ref)
    say(f"  {tag}: {excl}/{Hq} heads excluded as near-ties, output max abs {err:.2e}, rel L2 {r:.2e}")
    assert err <= BF16_ATOL and r < REL_L2


def _run(q, K, V, p, bs, dt, seq_lens=None, append_new=0, corrupt_tail=0):
    """q [B, Hq, D], K/V [B, Hkv, S, D] fp32 -> per-sequence checks."""
    ops = _ops()
    qd = torch.from_numpy(q).to(dt).to(DEV)
    kd = torch.from_numpy(K).to(dt).to(DEV)
    vd = torch.from_numpy(V).to(dt).to(DEV)
    sl = None if seq_lens is None else torch.tensor(seq_lens, dtype=torch.int32, device=DEV)
    est = p.get("est", "centroid")
    if corrupt_tail:
        # summaries built while the newest tokens still held other keys: the
        # step's append must recompute those blocks from the real keys
        kstale = kd.clone()
        kstale[:, :, K.shape[2] - corrupt_tail:] = 7.0
        c = ops.centroid_build(kstale, bs, seq_lens=sl, centroid_dtype=dt, estimator=est)
    else:
        c = ops.centroid_build(kd, bs, seq_lens=sl, centroid_dtype=dt, estimator=est)
    out, table, lens = ops.decode_fused(qd, kd, vd, c, bs, _budget(ops, p), seq_lens=sl,
                                        append_new=append_new, return_selection=True, estimator=est)
    torch.cuda.synchronize()
    if corrupt_tail:
        fresh = ops.centroid_build(kd, bs, seq_lens=sl, centroid_dtype=dt, estimator=est)
        torch.cuda.synchronize()
        assert torch.equal(c, fresh), "appended blocks' summaries differ from a rebuild"
    qr, Kr, Vr = _rounded(q, dt), _rounded(K, dt), _rounded(V, dt)
    c_np, table, lens, out = c.float().cpu().numpy(), table.cpu().numpy(), lens.cpu().numpy(), \
        out.float().cpu().numpy()
    for b in range(q.shape[0]):
        S_b = K.shape[2] if seq_lens is None else int(seq_lens[b])
        nb = -(-S_b // bs)
        if nb == 0:
            assert (lens[b] == 0).all() and np.isnan(out[b]).all()
            continue
        _check_sequence(qr[b], Kr[b][:, :S_b], Vr[b][:, :S_b], c_np[b][:, :nb], table[b], lens[b],
                        out[b], p, bs, f"sequence {b} ({S_b} tokens)")


GOLDEN = ["cfg1_seed0", "cfg1_seed2_fixed", "cfg1_seed3_avg32", "peaked_mixed", "partial_tail",
          "temp_sink_local", "gqa6_kmax256", "tiny_overlap", "single_block", "bs32", "planted",
          "kmin_above_floor", "kmax_below_floor", "large_budget"]


@pytest.mark.parametrize("name", GOLDEN)
def test_fused_bf16_golden_inputs(name):
    p = cases.params(name)
    say(f"fused bf16 {name}")
    q, K, V = cases.make_inputs(name)
    _run(q[None], K[None], V[None], p, p["bs"], torch.bfloat16)


@pytest.mark.parametrize("name", ["cfg1_seed0", "partial_tail", "temp_sink_local"])
def test_fused_fp16_golden_inputs(name):
    p = cases.params(name)
    say(f"fused fp16 {name}")
    q, K, V = cases.make_inputs(name)
    _run(q[None], K[None], V[None], p, p["bs"], torch.float16)


def _params(**kw):
    p = dict(policy="adaptive", temp=1.0, sink=1, local=4, cmin=1, kmin=2, kmax=64, avg=8)
    p.update(kw)
    return p


def _inputs(seed, B, Hq, Hkv, S, D, peaked=True):
    rng = np.random.RandomState(seed)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    if peaked:
        K[:, : Hkv // 2] *= np.float32(3.0)
    return q, K, V


@pytest.mark.parametrize("Hq,Hkv,D", [(64, 8, 64), (48, 8, 32), (40, 5, 128), (128, 8, 128), (32, 2, 64)])
def test_fused_many_heads(Hq, Hkv, D):
    """More q-heads than one merge pass covers (32 per pass); groups of 16
    q-heads per KV head (128 q / 8 KV heads, the largest group accepted)."""
    say(f"fused Hq={Hq} Hkv={Hkv} D={D}")
    q, K, V = _inputs(21, 1, Hq, Hkv, 4096, D)
    _run(q, K, V, _params(avg=10), 16, torch.bfloat16)


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_fused_group16_other_dtypes(dt):
    """Group 16 with fp32 K/V (the exact mode: its vector-unit scan and decode)
    and fp16, a ragged batch of two."""
    say(f"fused 128 q / 8 KV heads, {dt}")
    q, K, V = _inputs(23, 2, 128, 8, 3000, 64)
    _run(q, K, V, _params(avg=12), 16, dt, seq_lens=[3000, 1777])


def test_group16_plan_then_sparse_decode():
    """128 q / 8 KV heads through plan + table-driven decode: the plan's
    selection against the oracle and the decode against fp64 attention over it."""
    ops = _ops()
    say("plan + sparse decode, 128 q / 8 KV heads")
    q, K, V = _inputs(27, 1, 128, 8, 6000, 128)
    dt = torch.bfloat16
    qd, kd, vd = (torch.from_numpy(x).to(dt).to(DEV) for x in (q, K, V))
    c = ops.centroid_build(kd, 16, centroid_dtype=dt)
    budget = ops.BudgetParams(avg_budget=8)
    table, lens = ops.plan(qd, c, 16, budget, seq_len=6000)
    out = ops.sparse_decode(qd, kd, vd, table, lens, 16)
    torch.cuda.synchronize()
    _check_sequence(_rounded(q[0], dt), _rounded(K[0], dt), _rounded(V[0], dt), c[0].float().cpu().numpy(),
                    table[0].cpu().numpy(), lens[0].cpu().numpy(), out[0].float().cpu().numpy(),
                    _params(avg=8), 16, "plan + sparse decode")


@pytest.mark.parametrize("bs", [24, 32, 8])
def test_fused_block_sizes(bs):
    """Non-power-of-two block size (integer division), two 16-token tiles per block, half tiles."""
    say(f"fused block size {bs}")
    q, K, V = _inputs(22, 1, 16, 4, 3001, 128)
    _run(q, K, V, _params(avg=12), bs, torch.bfloat16)


def test_fused_append_several_rows():
    """append_new spanning three blocks: their centroids are recomputed from K by the step."""
    say("fused append 40 tokens")
    q, K, V = _inputs(23, 1, 32, 8, 4096 + 7, 128)
    _run(q, K, V, _params(avg=8), 16, torch.bfloat16, append_new=40, corrupt_tail=40)


def test_scan_launch_alone_matches_the_step():
    """adakv_decode_fused_scan, the step's first launch alone: its append
    rewrites the stale newest blocks exactly as a rebuild, and the step that
    follows on the same summaries selects as the whole step does."""
    say("fused scan launch alone (append 40 tokens)")
    ops = _ops()
    q, K, V = _inputs(26, 1, 32, 8, 4096 + 7, 128)
    qd, kd, vd = (torch.from_numpy(x).to(torch.bfloat16).to(DEV) for x in (q, K, V))
    kstale = kd.clone()
    kstale[:, :, K.shape[2] - 40:] = 7.0
    c = ops.centroid_build(kstale, 16, centroid_dtype=torch.bfloat16)
    budget = _budget(ops, _params(avg=8))
    ops.decode_fused_scan(qd, kd, vd, c, 16, budget, append_new=40)
    fresh = ops.centroid_build(kd, 16, centroid_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(c, fresh), "the scan launch's append differs from a rebuild"
    _, t1, l1 = ops.decode_fused(qd, kd, vd, c, 16, budget, append_new=40, return_selection=True)
    _, t2, l2 = ops.decode_fused(qd, kd, vd, fresh, 16, budget, append_new=0, return_selection=True)
    torch.cuda.synchronize()
    assert torch.equal(l1, l2)
    for h in range(l1.shape[1]):
        n = int(l1[0, h])
        assert torch.equal(t1[0, h, :n], t2[0, h, :n]), f"head {h}"


def test_fused_ragged_batch_with_empty_sequence():
    """Lengths 0, 1, 777 and 4096 in one batch: NaN rows and zero counts for the empty one."""
    say("fused ragged batch [0, 1, 777, 4096]")
    q, K, V = _inputs(24, 4, 16, 4, 4096, 128)
    _run(q, K, V, _params(avg=8), 16, torch.bfloat16, seq_lens=[0, 1, 777, 4096])


def test_fused_fixed_policy_and_temperature():
    say("fused fixed policy, temperature 0.6")
    q, K, V = _inputs(25, 2, 32, 8, 2048, 128)
    _run(q, K, V, _params(avg=9, policy="fixed"), 16, torch.bfloat16)
    _run(q, K, V, _params(avg=9, temp=0.6), 16, torch.bfloat16)


def test_fused_matches_plan_then_sparse_decode():
    """The fused step equals plan + table-driven decode on the same inputs, and
    the plan's selection matches the oracle.  512 blocks with k_max 64: the
    plan's 256-thread selection ranks more candidates than it has threads
    (every content block passes its threshold)."""
    ops = _ops()
    say("fused vs plan + sparse decode")
    q, K, V = _inputs(26, 1, 32, 8, 8192, 128)
    dt = torch.bfloat16
    qd, kd, vd = (torch.from_numpy(x).to(dt).to(DEV) for x in (q, K, V))
    c = ops.centroid_build(kd, 16, centroid_dtype=dt)
    budget = ops.BudgetParams(avg_budget=8)
    out_f, table_f, lens_f = ops.decode_fused(qd, kd, vd, c, 16, budget, return_selection=True)
    table_p, lens_p = ops.plan(qd, c, 16, budget, seq_len=8192)
    out_p = ops.sparse_decode(qd, kd, vd, table_p, lens_p, 16)
    torch.cuda.synchronize()
    lf, lp = lens_f[0].cpu().numpy(), lens_p[0].cpu().numpy()
    tf, tp = table_f[0].cpu().numpy(), table_p[0].cpu().numpy()
    same = [h for h in range(32) if lf[h] == lp[h] and set(tf[h, :lf[h]]) == set(tp[h, :lp[h]])]
    say(f"  {len(same)}/32 heads with identical selections")
    assert len(same) >= 28
    of, op = out_f[0].float().cpu().numpy(), out_p[0].float().cpu().numpy()
    assert np.abs(of[same] - op[same]).max() <= 1e-2
    p = _params(avg=8)
    _check_sequence(_rounded(q[0], dt), _rounded(K[0], dt), _rounded(V[0], dt), c[0].float().cpu().numpy(),
                    tp, lp, op, p, 16, "plan + sparse decode")
