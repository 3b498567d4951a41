"""Comparison of an oracle implementation against the golden fixtures.

Kept separate from the test module so the mutation tests can run the same
checks against deliberately broken copies of the oracle.
"""
from __future__ import annotations

import os

import numpy as np

import cases

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# einsum accumulation order is a NumPy SIMD detail; on a different host CPU the
# last bits may move.  Scores / outputs are held to these bounds (relative to
# the largest magnitude), integer results (k, mask, counts) to equality.
SCORE_RTOL = 2e-6
OUT_ATOL = 2e-5


def load(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    if "mask" in d:
        shape = tuple(int(x) for x in d["mask_shape"])
        d["mask"] = np.unpackbits(d["mask"], axis=1)[:, : shape[1]].astype(bool)
    return d


def check_case(O, name: str) -> list[str]:
    """Run oracle module ``O`` on case ``name``; return a list of mismatches."""
    p = cases.params(name)
    g = load(name)
    q, Kkv, Vkv = cases.make_inputs(name)
    errs: list[str] = []
    if str(g["digest"]) != cases.input_digest(q, Kkv, Vkv):
        return [f"{name}: input digest drift (RandomState stream changed?)"]
    K, V = O.expand_gqa(Kkv, p["hq"]), O.expand_gqa(Vkv, p["hq"])
    r = O.sparse_attention(q, K, V, block_size=p["bs"], avg_budget=p["avg"], k_min=p["kmin"],
                           k_max=p["kmax"], estimator=p["est"], n_sink_blocks=p["sink"],
                           n_local_blocks=p["local"], c_min=p["cmin"],
                           budget_policy=p["policy"], return_all=True)
    scale = float(np.abs(g["scores"]).max()) or 1.0
    if r["scores"].shape != g["scores"].shape or \
            np.abs(r["scores"] - g["scores"]).max() > SCORE_RTOL * scale:
        errs.append(f"{name}: scores differ")
    if not np.array_equal(r["mask"], g["mask"]):
        errs.append(f"{name}: mask differs ({int((r['mask'] != g['mask']).sum())} blocks)")
    if not np.array_equal(r["counts"], g["counts"]):
        errs.append(f"{name}: counts differ")
    if "k" in g and not np.array_equal(r["k"], g["k"]):
        errs.append(f"{name}: budgets differ {r['k'][:8]} vs {g['k'][:8]}")
    if "k_temp" in g:
        nb = g["scores"].shape[1]
        kt = O.allocate_budget(g["scores"], p["avg"], min(p["kmin"], nb), min(p["kmax"], nb),
                               temperature=p["temp"], policy=p["policy"],
                               floor=min(p["sink"], nb) + min(p["local"], nb) + p["cmin"])
        if not np.array_equal(kt, g["k_temp"]):
            errs.append(f"{name}: temperature budgets differ")
    if "w" in g:
        w = O.budget_weights(g["scores"], p["policy"], p["temp"], 0.9)
        if w.dtype != np.float64 or not np.allclose(w, g["w"], rtol=1e-6, atol=0):
            errs.append(f"{name}: weights differ / dtype {w.dtype}")
    oscale = max(float(np.abs(g["out"]).max()), 1.0)
    if not np.all(np.isfinite(r["out"])) or \
            np.abs(r["out"].astype(np.float64) - g["out"]).max() > OUT_ATOL * oscale:
        errs.append(f"{name}: output differs")
    if "centroid_sum" in g:
        cs = r["summ"]["centroid"].astype(np.float64).sum(axis=(1, 2))
        if not np.allclose(cs, g["centroid_sum"], rtol=1e-9, atol=1e-9):
            errs.append(f"{name}: centroid checksum differs")
    return errs
