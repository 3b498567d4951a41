"""Write the golden fixtures from the real reference (run in the build container only).

    python tests/golden/make_golden.py [/path/to/reference]

Imports the reference's pure-NumPy oracle modules (``adakv.reference``,
``adakv.estimator``, ``adakv.budget``) and its torch planner
(``adakv.attention.plan_selection``) from the read-only reference checkout and
records, per case of ``cases.py``, the outputs whose exact bits nothing else
pins: fp32 einsum scores (estimator.py:74), entropy / nucleus weights
(budget.py:28-42), the round-half-even budgets (budget.py:85), the selection
mask and counts (selector.py:18-60) and the fp32 attention output
(reference.py:76-80).  Inputs are regenerated from seeds; only their sha256 is
stored.  The fixtures are data; no reference source is copied.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import cases  # noqa: E402


def main(ref_root: str = "/root/reference") -> None:
    sys.path.insert(0, ref_root)
    from adakv import budget as R_budget  # noqa: E402
    from adakv import estimator as R_est  # noqa: E402
    from adakv import reference as R  # noqa: E402
    assert os.path.abspath(R.__file__).startswith(os.path.abspath(ref_root)), R.__file__

    for name in cases.CASES:
        p = cases.params(name)
        q, Kkv, Vkv = cases.make_inputs(name)
        K = R.expand_gqa(Kkv, p["hq"])
        V = R.expand_gqa(Vkv, p["hq"])
        out, counts, mask = R.sparse_attention(
            q, K, V, block_size=p["bs"], avg_budget=p["avg"], k_min=p["kmin"], k_max=p["kmax"],
            estimator=p["est"], n_sink_blocks=p["sink"], n_local_blocks=p["local"],
            c_min=p["cmin"], budget_policy=p["policy"], return_mask=True)
        summ = R_est.build_block_summaries(K, p["bs"], p["est"])
        scores = R_est.block_scores(q, summ)
        nb = summ["n_blocks"]
        rec = dict(out=out.astype(np.float32), counts=counts.astype(np.int64),
                   mask=np.packbits(mask, axis=1), mask_shape=np.array(mask.shape),
                   scores=scores.astype(np.float32), digest=np.array(cases.input_digest(q, Kkv, Vkv)))
        if p["temp"] == 1.0:
            k = R_budget.allocate_budget(
                scores, p["avg"], min(p["kmin"], nb), min(p["kmax"], nb), policy=p["policy"],
                floor=min(p["sink"], nb) + min(p["local"], nb) + p["cmin"])
            rec["k"] = k.astype(np.int64)
        else:
            # the oracle entry point has no temperature; record the allocator at T directly
            k = R_budget.allocate_budget(
                scores, p["avg"], min(p["kmin"], nb), min(p["kmax"], nb), temperature=p["temp"],
                policy=p["policy"], floor=min(p["sink"], nb) + min(p["local"], nb) + p["cmin"])
            rec["k_temp"] = k.astype(np.int64)
        if p["policy"] != "fixed" and nb > 1:
            rec["w"] = np.asarray(R_budget._weights(scores, p["policy"], p["temp"], 0.9),
                                  dtype=np.float64)
        if p["est"] == "centroid":
            rec["centroid_sum"] = summ["centroid"].astype(np.float64).sum(axis=(1, 2))
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **rec)
        print(f"{name}: nb={nb} k[:8]={k[:8].tolist()} counts mean={counts.mean():.2f}")

    # Runtime planner format (attention.py:149-247): forced blocks first, then
    # content by descending score; sel_lens = k.  Recorded on CPU fp32 tensors.
    import torch  # noqa: E402
    from adakv.attention import AdaKVCache, plan_selection  # noqa: E402
    for name in ("cfg1_seed0", "gqa6_kmax256"):
        p = cases.params(name)
        q, Kkv, Vkv = cases.make_inputs(name)
        cache = AdaKVCache(block_size=p["bs"]).append_prefill(torch.from_numpy(Kkv),
                                                              torch.from_numpy(Vkv))
        bt, sl = plan_selection(torch.from_numpy(q), cache, p["avg"], k_min=p["kmin"],
                                k_max=p["kmax"], n_sink_blocks=p["sink"],
                                n_local_blocks=p["local"], c_min=p["cmin"],
                                budget_policy=p["policy"])
        np.savez_compressed(os.path.join(HERE, f"plan_{name}.npz"),
                            block_table=bt.numpy(), sel_lens=sl.numpy())
        print(f"plan_{name}: table {tuple(bt.shape)} sel_lens[:8]={sl[:8].tolist()}")


if __name__ == "__main__":
    main(*sys.argv[1:])
