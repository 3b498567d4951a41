"""The reference-named wrappers on the GPU, called the way the reference's own
tests call them:

* ``adakv.kernels.block_sparse_decode.block_sparse_decode`` with the 3-D
  signature after ``plan_selection`` on an ``AdaKVCache``, at the two shapes
  of tests/test_kernel_parity.py:46-69, against attention over the same
  table (the oracle's ``ref_from_table``, fp64);
* ``adakv.runtime.update_cache_decode`` over 50 appends against a rebuild
  from the whole cache (tests/test_runtime_cpu.py:34-44);
* a 20-step ``update_cache_decode`` + ``adakv_decode_step`` loop at full
  budget against dense attention over the cache (tests/test_runtime_cpu.py:76-93).
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import DEV, need_gpu, rel_l2, say, torch
from oracle import adakv_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    need_gpu()


def _dense_one(qh, k, v, group, D):
    """Dense fp64 attention of one query per head over the whole cache: qh [Hq, D], k/v [Hkv, S, D]."""
    q64, k64, v64 = (x.double().cpu().numpy() for x in (qh, k, v))
    out = np.zeros((q64.shape[0], D))
    for h in range(q64.shape[0]):
        s = k64[h // group] @ q64[h] / np.sqrt(D)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ v64[h // group]
    return out


@pytest.mark.parametrize("Hkv,group,S,D,bs", [(8, 4, 4096, 128, 16), (4, 1, 8192, 64, 32)])
def test_block_sparse_decode_3d_matches_reference(Hkv, group, S, D, bs):
    from adakv.attention import AdaKVCache, plan_selection
    from adakv.kernels.block_sparse_decode import block_sparse_decode
    say(f"block_sparse_decode 3-D: Hkv {Hkv} group {group} S {S} D {D} bs {bs}, fp16")
    torch.manual_seed(0)
    Hq = Hkv * group
    q = torch.randn(Hq, D, device=DEV, dtype=torch.float16)
    k = torch.randn(Hkv, S, D, device=DEV, dtype=torch.float16) * 0.1
    v = torch.randn(Hkv, S, D, device=DEV, dtype=torch.float16)
    cache = AdaKVCache(block_size=bs).append_prefill(k, v)
    block_table, sel_lens = plan_selection(q, cache, avg_budget=16, k_min=2, k_max=64)
    out = block_sparse_decode(q, cache.k, cache.v, block_table, sel_lens, bs)
    torch.cuda.synchronize()
    assert out.shape == (Hq, D) and out.dtype == torch.float16
    ref = O.ref_from_table(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                           block_table.cpu().numpy(), sel_lens.cpu().numpy(), bs, group)
    r = rel_l2(out.float().cpu().numpy(), ref)
    say(f"  rel L2 {r:.2e}, sel_lens mean {sel_lens.float().mean().item():.1f}")
    assert r < 2e-3


def test_update_cache_decode_50_appends_equals_rebuild():
    from adakv.attention import AdaKVCache
    from adakv.runtime import update_cache_decode
    say("update_cache_decode: 50 appends from 100 tokens == rebuild")
    torch.manual_seed(0)
    Hkv, S0, D, bs = 4, 100, 32, 16          # a partial last block to start with
    cache = AdaKVCache(block_size=bs).append_prefill(torch.randn(Hkv, S0, D, device=DEV),
                                                     torch.randn(Hkv, S0, D, device=DEV))
    for _ in range(50):
        update_cache_decode(cache, torch.randn(Hkv, 1, D, device=DEV), torch.randn(Hkv, 1, D, device=DEV))
    rebuilt = AdaKVCache(block_size=bs).append_prefill(cache.k.clone(), cache.v.clone())
    torch.cuda.synchronize()
    assert cache.seq_len == S0 + 50 and cache.centroid.shape == rebuilt.centroid.shape
    # the append recomputes the touched blocks from K exactly as the build does
    assert torch.equal(cache.centroid, rebuilt.centroid)


def test_decode_step_loop_full_budget_equals_dense():
    from adakv.attention import AdaKVCache
    from adakv.runtime import adakv_decode_step, update_cache_decode
    say("adakv_decode_step: 20 steps at full budget == dense")
    torch.manual_seed(3)
    Hkv, group, S0, D, bs = 4, 2, 200, 64, 16
    Hq = Hkv * group
    cache = AdaKVCache(block_size=bs).append_prefill(torch.randn(Hkv, S0, D, device=DEV) * 0.1,
                                                     torch.randn(Hkv, S0, D, device=DEV))
    for _ in range(20):
        update_cache_decode(cache, torch.randn(Hkv, 1, D, device=DEV) * 0.1, torch.randn(Hkv, 1, D, device=DEV))
        q = torch.randn(1, Hq, 1, D, device=DEV)
        nb = cache.centroid.shape[1]
        out = adakv_decode_step(q, cache, avg_budget=nb, k_min=nb, k_max=nb)
        assert out.shape == (1, Hq, 1, D)
        dense = _dense_one(q[0, :, 0, :], cache.k, cache.v, group, D)
        r = rel_l2(out[0, :, 0, :].double().cpu().numpy(), dense)
        assert r < 1e-4, f"step decode != dense: rel {r:.2e}"


@pytest.mark.parametrize("name", ["cfg1_seed0", "gqa6_kmax256"])
def test_plan_selection_table_width_is_max_sel_lens(name):
    """``plan_selection`` returns the reference's table width, max(sel_lens)
    (adakv/attention.py:242-244), on the inputs of the reference's own planner
    fixtures (tests/golden/plan_*.npz, written by the reference): its rows are
    the static-width plan's, its selection is the reference's (near-ties
    excluded and counted), and with none excluded its shape and selected sets
    are the golden table's."""
    import os
    import cases
    import golden_check
    from gpu_util import compare_selection
    from adakv.attention import AdaKVCache, _budget, _validate, plan_selection
    from adakv_amd import ops
    say(f"plan_selection table width: {name}")
    p = cases.params(name)
    q, Kkv, Vkv = cases.make_inputs(name)
    with np.load(os.path.join(golden_check.GOLDEN, f"plan_{name}.npz")) as z:
        gbt, gsl = z["block_table"], z["sel_lens"]
    g = golden_check.load(name)
    cache = AdaKVCache(block_size=p["bs"]).append_prefill(torch.from_numpy(Kkv).to(DEV),
                                                          torch.from_numpy(Vkv).to(DEV))
    qd = torch.from_numpy(q).to(DEV)
    bt, sl = plan_selection(qd, cache, p["avg"], k_min=p["kmin"], k_max=p["kmax"], n_sink_blocks=p["sink"],
                            n_local_blocks=p["local"], c_min=p["cmin"], budget_policy=p["policy"])
    budget = _budget(p["avg"], p["kmin"], p["kmax"], p["sink"], p["local"], 1.0, p["policy"], p["cmin"])
    full, flens = ops.plan(qd.unsqueeze(0), _validate(cache, "centroid", p["policy"]), cache.block_size, budget,
                           seq_len=cache.seq_len)
    torch.cuda.synchronize()
    bt, sl, full, flens = bt.cpu().numpy(), sl.cpu().numpy(), full[0].cpu().numpy(), flens[0].cpu().numpy()
    assert bt.dtype == np.int32 and bt.flags["C_CONTIGUOUS"]
    assert bt.shape == (q.shape[0], int(sl.max()))
    assert full.shape[1] >= bt.shape[1] and np.array_equal(flens, sl)
    assert np.array_equal(full[:, : bt.shape[1]], bt)
    nb = g["scores"].shape[1]
    lo, hi, target, _ = O.budget_bounds(nb, p["avg"], p["kmin"], p["kmax"], p["sink"], p["local"], p["cmin"])
    excl = compare_selection(g["scores"], bt, sl, k_oracle=g["k"], w_oracle=g.get("w", np.ones(q.shape[0])),
                             lo=lo, target=target, sink=p["sink"], local=p["local"], cmin=p["cmin"],
                             policy=p["policy"])
    say(f"  width {bt.shape[1]} (golden {gbt.shape[1]}), {excl} near-tie heads excluded")
    if excl == 0:
        assert bt.shape == gbt.shape and np.array_equal(sl, gsl)
        for h in range(bt.shape[0]):
            n = int(sl[h])
            assert set(bt[h, :n].tolist()) == set(gbt[h, :n].tolist()), f"head {h}"
