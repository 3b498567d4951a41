"""Seeded input generators for the golden fixtures (shared by the fixture
writer and the tests, so the fixtures store only small outputs + an input hash).

``np.random.RandomState`` is a frozen stream (NEP 19), so the inputs are
reproducible on every machine; the sha256 stored with each fixture detects
any drift.
"""
from __future__ import annotations

import hashlib

import numpy as np

# name -> parameters.  "hkv"/"hq" heads, "d" head_dim, "s" tokens, "bs" block size.
# kscale multiplies K; "peaked" scales the keys of the first half of the KV heads
# so their block-score softmax is sharper; "plant" plants q-aligned blocks
# (tests/test_reference.py:24-32 pattern) in every KV head.
CASES = {
    # 32 q / 8 KV heads, D 128, S 4096, bs 16, avg 8, fp32 N(0,1), RandomState(0) q,K,V
    "cfg1_seed0": dict(seed=0, hq=32, hkv=8, d=128, s=4096, bs=16, avg=8),
    "cfg1_seed1": dict(seed=1, hq=32, hkv=8, d=128, s=4096, bs=16, avg=8),
    "cfg1_seed2_fixed": dict(seed=2, hq=32, hkv=8, d=128, s=4096, bs=16, avg=8, policy="fixed"),
    "cfg1_seed3_avg32": dict(seed=3, hq=32, hkv=8, d=128, s=4096, bs=16, avg=32),
    "peaked_mixed": dict(seed=4, hq=32, hkv=8, d=128, s=2048, bs=16, avg=8, peaked=True),
    "partial_tail": dict(seed=5, hq=8, hkv=2, d=64, s=4001, bs=16, avg=8),
    "temp_sink_local": dict(seed=6, hq=8, hkv=4, d=64, s=1024, bs=16, avg=12, temp=0.5,
                            sink=2, local=3, cmin=2),
    "gqa6_kmax256": dict(seed=7, hq=12, hkv=2, d=64, s=320, bs=16, avg=8, kmax=256,
                         sink=1, local=2, cmin=1),
    "tiny_overlap": dict(seed=8, hq=4, hkv=2, d=32, s=40, bs=16, avg=8),
    "single_block": dict(seed=9, hq=4, hkv=1, d=32, s=12, bs=16, avg=8),
    "bs32": dict(seed=10, hq=8, hkv=4, d=64, s=8192, bs=32, avg=16),
    "planted": dict(seed=11, hq=8, hkv=2, d=64, s=512, bs=16, avg=6, kscale=0.1, plant=(7,),
                    local=2),
    "kmin_above_floor": dict(seed=12, hq=8, hkv=2, d=64, s=1024, bs=16, avg=10, kmin=9),
    "kmax_below_floor": dict(seed=13, hq=8, hkv=2, d=64, s=1024, bs=16, avg=8, kmax=3),
    "large_budget": dict(seed=14, hq=8, hkv=2, d=64, s=2048, bs=16, avg=100, kmax=100000),
    "nucleus": dict(seed=15, hq=16, hkv=4, d=64, s=2048, bs=16, avg=8, policy="adaptive_nucleus"),
    "minmax_fixed": dict(seed=16, hq=16, hkv=4, d=64, s=2048, bs=16, avg=8, est="minmax",
                         policy="fixed"),
}


def params(name: str) -> dict:
    p = dict(policy="adaptive", temp=1.0, sink=1, local=4, cmin=1, kmin=2, kmax=64,
             est="centroid", kscale=1.0, peaked=False, plant=())
    p.update(CASES[name])
    return p


def make_inputs(name: str):
    """Returns q [Hq,D], K [Hkv,S,D], V [Hkv,S,D] as float32 (draw order q, K, V)."""
    p = params(name)
    rng = np.random.RandomState(p["seed"])
    q = rng.standard_normal((p["hq"], p["d"])).astype(np.float32)
    K = rng.standard_normal((p["hkv"], p["s"], p["d"])).astype(np.float32)
    V = rng.standard_normal((p["hkv"], p["s"], p["d"])).astype(np.float32)
    if p["kscale"] != 1.0:
        K *= np.float32(p["kscale"])
    if p["peaked"]:
        K[: p["hkv"] // 2] *= np.float32(4.0)
    g = p["hq"] // p["hkv"]
    for blk in p["plant"]:
        lo = blk * p["bs"]
        for h in range(p["hkv"]):
            K[h, lo:lo + p["bs"]] = q[h * g][None, :] * np.float32(3.0)
    return q, K, V


def input_digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()
