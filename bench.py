#!/usr/bin/env python3
"""AdaKV decode-attention benchmark on one MI355X.

Workload (N=1): one Llama-3.1-8B-shaped attention layer
decoding one token -- batch 1, 32 q / 8 KV heads, head_dim 128, context
131072, bf16 K/V ~ N(0,1), block_size 16, avg_budget 8 (adaptive entropy
budget, sink 1, local 4, c_min 1, k_max 64).  Every KV head holds 4 planted
"needle" blocks whose keys are 3 * q + noise for one of its q-heads.

A step is one layer's full decode-attention op: centroid append for the new
token, block scores, budget + selection, sparse split-K decode and merge
(adakv_decode_fused).  Steps cycle over ``--layers`` independent layers'
K/V/centroid buffers (32 by default: 16 GiB of K/V, 512 MiB of centroids,
more than the 256 MB MALL) so every step reads HBM.  Launches are captured in
a HIP graph to take host overhead out: exactly --warmup untimed layer-steps,
then exactly --steps timed ones.

Prints one JSON line: value = microseconds per layer (lower is better), the
achieved HBM GB/s on the algorithmic bytes of the op, the dense HIP
flash-decode time at the same context, the rooflines of the step's two
launches (the scan launch timed alone with HIP events exactly as the step
issues it; the select + decode launch as the rest of the step), and the CPU
oracle timed on one
layer of the same workload on this host.  ``cells`` holds the other methods of
the reference's decode-latency table (benchmarks/efficiency/
bench_decode_latency.py:11-19) on the same layers at the same avg_budget:
quest (minmax bounds + fixed budget), adakv_cf (centroids + fixed budget),
adakv_nucleus (centroids + the nucleus budget, the cell that table labels
"adakv"), streaming (sink + most recent blocks, no scoring) and dense, with
each estimator's summary bytes per layer.  ``eviction`` holds the H2O /
SnapKV baselines (adakv/baselines_rt.py): the prefill-side key importance
against its roofline and the reference's torch formulation, the retention,
and the frozen decode step on the same layers.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

PEAK_HBM_GBPS = 8000.0
PEAK_BF16_TFLOPS = 2500.0          # dense bf16 matrix-core peak
METRIC = "decode attn µs/layer @128K + achieved HBM GB/s (KV bytes touched), 1 MI355X"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640, help="timed layer-steps of the headline (exactly)")
    ap.add_argument("--warmup", type=int, default=64, help="untimed layer-steps")
    ap.add_argument("--ctx", type=int, default=131072)
    ap.add_argument("--avg-budget", type=float, default=8)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="CPU-oracle time budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--no-cells", action="store_true", help="skip the quest / adakv_cf / streaming legs")
    ap.add_argument("--no-sweep", action="store_true", help="skip the context sweep")
    ap.add_argument("--no-ragged", action="store_true", help="skip the ragged-batch leg (BASELINE config 4)")
    ap.add_argument("--sweep-ctx", type=str, default="4096,16384,32768,65536,262144")
    ap.add_argument("--no-evict", action="store_true", help="skip the H2O / SnapKV eviction-baseline legs")
    ap.add_argument("--h2o-len", type=int, default=8192, help="prompt length of the H2O importance leg")
    ap.add_argument("--model-step", action="store_true",
                    help="BASELINE config 5 instead: a Llama-3-70B-shaped 80-layer decode step through patch_model")
    ap.add_argument("--no-model-step", action="store_true",
                    help="skip the config-5 model-step leg of the default run")
    ap.add_argument("--model-layers", type=int, default=80)
    ap.add_argument("--model-batch", type=int, default=4)
    ap.add_argument("--model-ctx", type=int, default=65536)
    ap.add_argument("--seed", type=int, default=0)
    return ap.parse_args()


class Workload:
    Hq, Hkv, D, BS = 32, 8, 128, 16

    def __init__(self, torch, ops, ctx, layers, avg_budget, seed):
        self.torch, self.ops = torch, ops
        self.S, self.L = ctx, layers
        self.nb = ops.n_blocks(ctx, self.BS)
        self.budget = ops.BudgetParams(avg_budget=avg_budget)
        dev = torch.device("cuda:0")
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        G = self.Hq // self.Hkv
        self.q, self.k, self.v, self.c, self.out, self.needles = [], [], [], [], [], []
        rng = torch.Generator().manual_seed(seed)
        for _ in range(layers):
            q = torch.randn(1, self.Hq, self.D, device=dev, dtype=torch.bfloat16, generator=gen)
            k = torch.randn(1, self.Hkv, ctx, self.D, device=dev, dtype=torch.bfloat16, generator=gen)
            v = torch.randn(1, self.Hkv, ctx, self.D, device=dev, dtype=torch.bfloat16, generator=gen)
            # 4 needle blocks per KV head at content positions (not sink, not local)
            pos = torch.randint(1, self.nb - 4, (self.Hkv, 4), generator=rng)
            for g in range(self.Hkv):
                for j in range(4):
                    b = int(pos[g, j])
                    lo, hi = b * self.BS, min((b + 1) * self.BS, ctx)
                    k[0, g, lo:hi] = (3.0 * q[0, g * G + j].float()[None, :] +
                                      torch.randn(hi - lo, self.D, device=dev, generator=gen)).to(torch.bfloat16)
            c = ops.centroid_build(k, self.BS)
            self.q.append(q)
            self.k.append(k)
            self.v.append(v)
            self.c.append(c)
            self.out.append(torch.empty(1, self.Hq, self.D, device=dev, dtype=torch.bfloat16))
            self.needles.append(pos)
        torch.cuda.synchronize()

    def step(self, l):
        self.ops.decode_fused(self.q[l], self.k[l], self.v[l], self.c[l], self.BS, self.budget,
                              append_new=1, out=self.out[l])

    def build_cells(self, avg_budget):
        """Minmax bounds per layer, the fixed budget, and a streaming table
        (bench_decode_latency.py:56-63: sink blocks + the most recent window)."""
        torch, ops = self.torch, self.ops
        self.m = [ops.centroid_build(k, self.BS, estimator="minmax") for k in self.k]
        self.fixed = ops.BudgetParams(avg_budget=avg_budget, budget_policy="fixed")
        self.nucleus = ops.BudgetParams(avg_budget=avg_budget, budget_policy="adaptive_nucleus")
        bud = int(round(avg_budget))
        sink = self.budget.n_sink_blocks
        win = max(bud - sink, 1)
        idx = torch.cat([torch.arange(0, sink), torch.arange(self.nb - win, self.nb)])[:bud]
        self.st_table = idx.to(torch.int32).view(1, 1, -1).expand(1, self.Hq, -1).contiguous().cuda()
        self.st_lens = torch.full((1, self.Hq), idx.numel(), dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()

    def quest(self, l):
        self.ops.decode_fused(self.q[l], self.k[l], self.v[l], self.m[l], self.BS, self.fixed,
                              append_new=1, out=self.out[l])

    def adakv_cf(self, l):
        self.ops.decode_fused(self.q[l], self.k[l], self.v[l], self.c[l], self.BS, self.fixed,
                              append_new=1, out=self.out[l])

    def adakv_nucleus(self, l):
        self.ops.decode_fused(self.q[l], self.k[l], self.v[l], self.c[l], self.BS, self.nucleus,
                              append_new=1, out=self.out[l])

    def streaming(self, l):
        self.ops.sparse_decode(self.q[l], self.k[l], self.v[l], self.st_table, self.st_lens, self.BS,
                               out=self.out[l])

    def minmax_scores(self, l, buf):
        self.ops.block_scores(self.q[l], self.m[l], self.BS, seq_len=self.S, out=buf)

    def dense(self, l):
        self.ops.dense_decode(self.q[l], self.k[l], self.v[l], out=self.out[l])

    def scores(self, l, buf):
        self.ops.block_scores(self.q[l], self.c[l], self.BS, seq_len=self.S, out=buf)

    def scan(self, l):
        """The step's first launch alone, as the step issues it."""
        self.ops.decode_fused_scan(self.q[l], self.k[l], self.v[l], self.c[l], self.BS, self.budget,
                                   append_new=1)


def capture(torch, fn, layers, stream):
    """One HIP graph holding fn(0..layers-1), after a warm pass on the capture stream."""
    with torch.cuda.stream(stream):
        for l in range(layers):
            fn(l)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for l in range(layers):
            fn(l)
    torch.cuda.synchronize()
    return g


def capture_steps(torch, fn, n, layers, stream):
    """One HIP graph of exactly n layer-steps fn(i % layers), i < n (the
    caller has run fn eagerly on `stream` once, so nothing allocates inside)."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(n):
            fn(i % layers)
    torch.cuda.synchronize()
    return g


def time_exact(torch, fn, steps, warmup, layers, stream):
    """Exactly `warmup` untimed layer-steps, then exactly `steps` timed ones
    (one graph replay bracketed by synchronisations, HIP events on the
    current stream).  The warm-up is an eager pass over the first
    min(warmup, layers) layers (it also allocates the workspace), then a
    graph of the rest.  Returns (ms, wall ms) of the timed steps."""
    eager = max(1, min(warmup, layers))
    with torch.cuda.stream(stream):
        for i in range(eager):
            fn(i % layers)
    torch.cuda.synchronize()
    g = capture_steps(torch, fn, steps, layers, stream)
    if warmup > eager:
        gw = capture_steps(torch, fn, warmup - eager, layers, stream)
        gw.replay()
        torch.cuda.synchronize()
        del gw
    ms, wall = time_graph(torch, g, 1, 0)
    del g
    return ms, wall


def time_graph(torch, g, replays, warm):
    """HIP-event time of `replays` graph replays on the current stream (ms)."""
    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    s.record()
    for _ in range(replays):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    return s.elapsed_time(e), wall


def selection_bytes(torch, ops, w: Workload):
    """Algorithmic bytes of one layer step, from the actual selection of every layer."""
    e = 2
    uniq = []
    for l in range(w.L):
        _, table, lens = ops.decode_fused(w.q[l], w.k[l], w.v[l], w.c[l], w.BS, w.budget,
                                          return_selection=True)
        t, n = table[0].cpu(), lens[0].cpu()
        G = w.Hq // w.Hkv
        u = 0
        for g in range(w.Hkv):
            s = set()
            for h in range(g * G, (g + 1) * G):
                s.update(t[h, : int(n[h])].tolist())
            u += len(s)
        uniq.append(u)
    u = sum(uniq) / len(uniq)
    T = ops.table_width(1, w.Hq, w.Hkv, w.D, w.BS, w.S, w.c[0].shape[2], w.budget)
    b_cent = w.Hkv * w.nb * w.D * e
    b_kv = u * w.BS * w.D * e * 2
    b_q = b_out = w.Hq * w.D * e
    b_meta = w.Hq * T * 4 * 2 + w.Hq * 4 * 2 + w.Hkv * (w.BS * w.D * e + w.D * e)
    return dict(centroid=b_cent, kv=b_kv, q=b_q, out=b_out, meta=b_meta,
                total=b_cent + b_kv + b_q + b_out + b_meta, union_blocks_per_layer=u)


def scan_bytes(w: Workload):
    """Algorithmic bytes of the step's scan launch at this shape: every
    centroid row and q read, the fp32 scores and the 80-byte softmax records
    (one per q-head and 256-row workgroup) written, and the centroid append
    of the newest token's block (its 16 K rows read, its row and its scores
    written)."""
    e = 2
    n_rec = w.Hq * ((w.nb + 255) // 256)
    parts = dict(centroid=w.Hkv * w.nb * w.D * e, q=w.Hq * w.D * e, scores=w.Hq * w.nb * 4,
                 records=n_rec * 80, append=w.Hkv * (w.BS * w.D * e + w.D * e) + w.Hq * 4)
    parts["total"] = sum(parts.values())
    return parts


def ragged_batch(torch, ops, stream, seed, layers=16):
    """8 sequences with lengths uniform in [16K, 128K] (fixed
    seed), 32 q / 8 KV heads, head_dim 128, bf16, block_size 16, avg_budget 16;
    half the KV heads peaked (keys x4).  One step decodes the whole batch
    (per-sequence lengths on the device); 16 layers' buffers rotate (their
    centroids, about 0.9 GB, exceed the 256 MB MALL, so every step reads HBM;
    K/V take 4 GiB per layer)."""
    B, Hq, Hkv, D, BS, cap = 8, 32, 8, 128, 16, 131072
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(seed)
    lens = torch.randint(16384, cap + 1, (B,), generator=torch.Generator().manual_seed(seed)).to(torch.int32)
    sl = lens.to(dev)
    budget = ops.BudgetParams(avg_budget=16)
    L = []
    for _ in range(layers):
        k = torch.randn(B, Hkv, cap, D, device=dev, dtype=torch.bfloat16, generator=gen)
        k[:, : Hkv // 2] *= 4.0
        v = torch.randn(B, Hkv, cap, D, device=dev, dtype=torch.bfloat16, generator=gen)
        q = torch.randn(B, Hq, D, device=dev, dtype=torch.bfloat16, generator=gen)
        c = ops.centroid_build(k, BS, seq_lens=sl)
        L.append((q, k, v, c, torch.empty_like(q)))
    torch.cuda.synchronize()

    def step(l):
        q, k, v, c, o = L[l]
        ops.decode_fused(q, k, v, c, BS, budget, seq_lens=sl, append_new=1, out=o)

    def dense(l):
        q, k, v, _, o = L[l]
        ops.dense_decode(q, k, v, seq_lens=sl, out=o)

    g1 = capture(torch, step, layers, stream)
    ms1, _ = time_graph(torch, g1, 10, 1)
    g2 = capture(torch, dense, layers, stream)
    ms2, _ = time_graph(torch, g2, 3, 1)
    a_us, d_us = ms1 * 1e3 / (10 * layers), ms2 * 1e3 / (3 * layers)
    kv_dense = int(lens.sum()) * Hkv * D * 2 * 2
    # AdaKV's algorithmic bytes per step, from each layer's own selection:
    # every sequence's centroid rows, each (sequence, KV head)'s union of
    # selected blocks (K and V), q and out, the tables and counts
    G = Hq // Hkv
    nbs = [(int(n) + BS - 1) // BS for n in lens.tolist()]
    b_cent = sum(nbs) * Hkv * D * 2
    unions = []
    for l in range(layers):
        q, k, v, c, _ = L[l]
        _, table, sel = ops.decode_fused(q, k, v, c, BS, budget, seq_lens=sl, return_selection=True)
        t, n = table.cpu(), sel.cpu()
        u = 0
        for b in range(B):
            for g in range(Hkv):
                s = set()
                for h in range(g * G, (g + 1) * G):
                    s.update(t[b, h, : int(n[b, h])].tolist())
                u += len(s)
        unions.append(u)
    u = sum(unions) / len(unions)
    b_kv = u * BS * D * 2 * 2
    b_qo = 2 * B * Hq * D * 2
    b_meta = B * Hq * (table.shape[2] + 1) * 4 * 2
    total = b_cent + b_kv + b_qo + b_meta
    gbps = total / (a_us * 1e-6) / 1e9
    log(f"ragged batch (config 4, lengths {lens.tolist()}): adakv {a_us:.2f} us/step ({gbps:.0f} GB/s), "
        f"dense {d_us:.2f} us/step")
    del g1, g2, L
    torch.cuda.empty_cache()
    return {"config": "BASELINE config 4: 8 sequences, lengths uniform in [16K, 128K], avg_budget 16",
            "lengths": lens.tolist(), "layers_rotated": layers, "adakv_us_per_layer_step": round(a_us, 2),
            "dense_us_per_layer_step": round(d_us, 2), "speedup": round(d_us / a_us, 2),
            "bytes_per_step": int(total), "centroid_bytes_per_step": int(b_cent),
            "kv_bytes_per_step": int(b_kv), "union_blocks_per_step": round(u, 1),
            "achieved_GBps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4),
            "dense_GBps": round(kv_dense / (d_us * 1e-6) / 1e9, 1),
            "dense_frac": round(kv_dense / (d_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}


def stream_copy_gbps(torch, nbytes: int = 1 << 30, reps: int = 10) -> float:
    """Measured device copy bandwidth (read + write bytes / time) of a plain
    torch copy of `nbytes`, the practical HBM ceiling next to the 8 TB/s peak."""
    x = torch.empty(nbytes // 4, device="cuda", dtype=torch.float32).fill_(1.0)
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        y.copy_(x)
    e.record()
    torch.cuda.synchronize()
    gbps = 2 * nbytes * reps / (s.elapsed_time(e) * 1e-3) / 1e9
    del x, y
    return gbps


def profiled_traffic(path: str):
    """HBM bytes per launch of the step's kernels, {kernel: bytes}, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (calibrated against a
    plain copy; lines `traffic_bytes_per_launch[kernel]: bytes`); None if absent."""
    out = {}
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch["):
                    name, val = line.split("]:", 1)
                    out[name[len("traffic_bytes_per_launch["):]] = int(val)
    except OSError:
        pass
    return out or None


def cpu_baseline(torch, w: Workload, budget_s: float):
    """The NumPy oracle (reference.sparse_attention restated) on layer 0 of the
    same workload, single-threaded NumPy einsum; median seconds per layer."""
    import numpy as np

    from oracle import adakv_oracle as O
    q = w.q[0][0].float().cpu().numpy()
    K = O.expand_gqa(w.k[0][0].float().cpu().numpy(), w.Hq)
    V = O.expand_gqa(w.v[0][0].float().cpu().numpy(), w.Hq)
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        O.sparse_attention(q, K, V, block_size=w.BS, avg_budget=w.budget.avg_budget)
        times.append(time.perf_counter() - t0)
        log(f"cpu oracle run {len(times)}: {times[-1]:.2f}s")
        if len(times) >= 5 or time.perf_counter() - t_start + times[-1] > budget_s:
            break
    del K, V
    runs = times[1:] if len(times) > 1 else times
    return float(np.median(runs)), len(times)


def time_calls(torch, fn, n, warm=1):
    """HIP-event time per call of fn() on the current stream (ms)."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(n):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / n


def torch_key_importance(torch, Q, K, first, chunk=256):
    """The reference runtime's formulation (adakv/baselines_rt.py:43-80): fp32
    logits per chunk of queries against every key, causal mask, softmax over
    keys, summed over the chunk -- torch ops on the same GPU, for comparison."""
    Hq, L, D = Q.shape
    G = Hq // K.shape[0]
    Kt = K.float().repeat_interleave(G, dim=0).transpose(1, 2).contiguous()      # [Hq, D, L]
    imp = torch.zeros(Hq, L, device=Q.device)
    keys = torch.arange(L, device=Q.device)
    for s0 in range(first, L, chunk):
        e0 = min(s0 + chunk, L)
        lg = torch.bmm(Q[:, s0:e0].float(), Kt) / math.sqrt(D)
        lg = lg.masked_fill(keys.view(1, 1, -1) > torch.arange(s0, e0, device=Q.device).view(1, -1, 1),
                            float("-inf"))
        imp += torch.softmax(lg, dim=-1).sum(dim=1)
    return imp


def evict_bench(torch, ops, w, stream, seed, h2o_len):
    """The eviction baselines (adakv/baselines_rt.py): the prefill-side
    importance (H2O over an h2o_len prompt, SnapKV's 32-query window over the
    headline 128K context) against the matrix-core and HBM rooflines and
    against the reference's torch formulation, the retention, and the frozen
    decode step on the headline workload."""
    from adakv import baselines_rt as BR
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    res = {}
    L = h2o_len
    Q = torch.randn(w.Hq, L, w.D, device=dev, dtype=torch.bfloat16, generator=gen)
    K = torch.randn(w.Hkv, L, w.D, device=dev, dtype=torch.bfloat16, generator=gen)
    ms = time_calls(torch, lambda: BR.key_importance(Q, K, 0), 5)
    ms_t = time_calls(torch, lambda: torch_key_importance(torch, Q, K, 0), 2)
    flops = 2 * w.Hq * (L * (L + 1) // 2) * 2 * w.D        # two passes over the causal (query, key) pairs
    tf = flops / (ms * 1e-3) / 1e12
    res["h2o_importance"] = {"prompt": L, "ms": round(ms, 3), "TFLOPs": round(tf, 1),
                             "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS,
                                          "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4)},
                             "torch_formulation_ms": round(ms_t, 2), "speedup_vs_torch": round(ms_t / ms, 1)}
    log(f"h2o importance, {L}-token prompt: {ms:.3f} ms ({tf:.0f} TFLOP/s useful); torch formulation {ms_t:.1f} ms")
    del Q, K
    S = w.S
    Qs = torch.randn(w.Hq, S, w.D, device=dev, dtype=torch.bfloat16, generator=gen)
    Ks = w.k[0][0]
    win = 32
    g_snap = capture(torch, lambda l: BR.snapkv_key_importance_torch(Qs, Ks, win, 7), 1, stream)
    ms_s, _ = time_graph(torch, g_snap, 20, 2)
    ms_s /= 20
    ms_st = time_calls(torch, lambda: torch_key_importance(torch, Qs, Ks, S - win), 3)
    sbytes = w.Hkv * S * w.D * 2 + w.Hq * win * w.D * 2 + w.Hq * S * 4 * 2   # K, window, importance (+pool)
    sg = sbytes / (ms_s * 1e-3) / 1e9
    res["snapkv_importance"] = {"prompt": S, "window": win, "pool": 7, "us": round(ms_s * 1e3, 1),
                                "GBps": round(sg, 1),
                                "roofline": {"bound": "hbm", "achieved": round(sg, 1), "peak": PEAK_HBM_GBPS,
                                             "unit": "GB/s", "frac": round(sg / PEAK_HBM_GBPS, 4),
                                             "bytes": int(sbytes)},
                                "torch_formulation_us": round(ms_st * 1e3, 1),
                                "speedup_vs_torch": round(ms_st / ms_s, 1)}
    log(f"snapkv importance, {S}-token prompt: {ms_s * 1e3:.1f} us ({sg:.0f} GB/s); "
        f"torch formulation {ms_st * 1e3:.0f} us")
    del g_snap
    imp = BR.snapkv_key_importance_torch(Qs, Ks, win, 7)
    del Qs
    ms_r = time_calls(torch, lambda: BR.retain_blocks_table(imp, w.BS, S, 8, 1, 4, 1), 20)
    res["retain_us"] = round(ms_r * 1e3, 1)
    log(f"retain ({w.nb} blocks x {w.Hq} heads): {ms_r * 1e3:.1f} us")
    frozen = []
    for l in range(w.L):
        r = torch.rand(w.Hq, S, device=dev, generator=gen)
        _, t, n = BR.retain_blocks_table(r, w.BS, S, 8, 1, 4, 1)
        frozen.append((t, n))

    def frozen_step(l):
        t, n = BR.frozen_table(frozen[l][0], frozen[l][1], w.nb, w.nb, 1, 4)
        ops.sparse_decode(w.q[l], w.k[l], w.v[l], t[None], n[None], w.BS, out=w.out[l])

    g_f = capture(torch, frozen_step, w.L, stream)
    ms_f, _ = time_graph(torch, g_f, 8, 1)
    res["frozen_decode_us_per_layer"] = round(ms_f * 1e3 / (8 * w.L), 3)
    log(f"frozen decode (table + sparse decode): {res['frozen_decode_us_per_layer']:.2f} us/layer")
    del g_f, imp, frozen
    torch.cuda.empty_cache()
    return res


def model_step(args):
    """Llama-3-70B-shaped decode (80 layers, hidden 8192, 64 q / 8 KV
    heads, head_dim 128, MLP 28672, vocab 128256) with random-init bf16 weights, batch 4,
    a 65536-token static KV cache synthesised directly (random bf16 K/V, no prefill),
    through ``patch_model`` (block_size 16, avg_budget 8).  Per-token decode latency with
    AdaKV, with a dense decode (this build's HIP flash-decode over every cached token, and
    HF's SDPA, which expands K/V per layer under the static cache's mask), and with the
    attention replaced by a no-op (which keeps the KV-cache write), so attention share
    = 1 - t_noop / t."""
    import torch
    from transformers import AttentionInterface, LlamaConfig, LlamaForCausalLM, StaticCache
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, sdpa_mask

    from adakv_amd import ops
    from adakv import patch as P
    dev = torch.device("cuda:0")
    L, B, S0 = args.model_layers, args.model_batch, args.model_ctx
    cfg = LlamaConfig(vocab_size=128256, hidden_size=8192, intermediate_size=28672, num_hidden_layers=L,
                      num_attention_heads=64, num_key_value_heads=8, head_dim=128,
                      max_position_embeddings=131072, rope_theta=500000.0, tie_word_embeddings=False)
    log(f"model step: {L} layers, batch {B}, ctx {S0}: building random-init bf16 weights on the GPU")
    with torch.device("meta"):
        model = LlamaForCausalLM(cfg)
    model = model.to(torch.bfloat16).to_empty(device=dev)        # bf16 before any memory exists
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    for i, (name, p) in enumerate(model.named_parameters()):
        with torch.no_grad():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, 0.02, generator=gen)
        if i % 9 == 0:
            log(f"  initialised {i} parameter tensors ({name})")
    # the rotary table is a non-persistent buffer: rebuild it on the device
    model.model.rotary_emb = type(model.model.rotary_emb)(config=cfg).to(dev)
    model.eval()
    P.install_adakv(model)
    n_params = sum(p.numel() for p in model.parameters())
    steps, warm = max(args.steps // 64, 4), 2
    cache = StaticCache(config=cfg, max_cache_len=S0 + 4 * (steps + warm) + 16)
    kd = torch.zeros(B, 8, 1, 128, dtype=torch.bfloat16, device=dev)
    for i, layer in enumerate(cache.layers):
        layer.lazy_initialization(kd, kd)
        layer.keys[:, :, :S0].normal_(generator=gen)
        layer.values[:, :, :S0].normal_(generator=gen)
        if isinstance(layer.cumulative_length, torch.Tensor):
            layer.cumulative_length.fill_(S0)
        else:
            layer.cumulative_length = S0
        if i % 4 == 0:
            log(f"  KV cache layer {i} filled")
    torch.cuda.synchronize()
    log(f"  {n_params / 1e9:.1f} B parameters, {torch.cuda.memory_allocated() / 2**30:.0f} GiB allocated")

    def noop_attention(module, query, key, value, attention_mask, scaling, dropout=0.0, **kw):
        Bq, Hq, q_len, D = query.shape
        return query.new_zeros(Bq, q_len, Hq, D), None

    def dense_hip_attention(module, query, key, value, attention_mask, scaling, dropout=0.0, **kw):
        Bq, Hq, q_len, D = query.shape
        runs = None if attention_mask is None else P._mask_runs(attention_mask, Bq, key.shape[2])
        if attention_mask is not None and (runs is None or any(runs[0])):
            raise RuntimeError("dense HIP leg: the static cache's mask is not a prefix per sequence")
        out = torch.empty(Bq, 1, Hq, D, dtype=query.dtype, device=query.device)
        ops.dense_decode(query[:, :, 0, :], key, value, sm_scale=scaling,
                         seq_lens=None if runs is None else runs[2], out=out[:, 0])
        return out, None

    AttentionInterface.register("adakv_noop", noop_attention)
    ALL_MASK_ATTENTION_FUNCTIONS.register("adakv_noop", sdpa_mask)
    AttentionInterface.register("adakv_dense_hip", dense_hip_attention)
    ALL_MASK_ATTENTION_FUNCTIONS.register("adakv_dense_hip", sdpa_mask)
    pos = [S0]

    def one_step():
        tok = torch.randint(0, cfg.vocab_size, (B, 1), device=dev, generator=gen)
        pid = torch.full((B, 1), pos[0], dtype=torch.long, device=dev)
        with torch.no_grad():
            model(input_ids=tok, position_ids=pid, past_key_values=cache, use_cache=True)
        pos[0] += 1

    def timed(label):
        for _ in range(warm):
            one_step()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(steps):
            one_step()
        e.record()
        torch.cuda.synchronize()
        ms = s.elapsed_time(e) / steps
        log(f"  {label}: {ms:.2f} ms/token")
        return ms

    P.enable_adakv(block_size=16, avg_budget=8, k_min=2, k_max=64, n_sink_blocks=1, n_local_blocks=4,
                   temperature=1.0, estimator="centroid", budget_policy="adaptive", c_min=1)
    t_adakv = timed("adakv (patch_model, avg_budget 8)")
    P.disable_adakv()
    t_dense = timed("dense (HF SDPA)")
    model.set_attn_implementation("adakv_dense_hip")
    t_dense_hip = timed("dense (HIP flash-decode)")
    model.set_attn_implementation("adakv_noop")
    t_noop = timed("attention replaced by a no-op")
    P.install_adakv(model)
    res = {
        "metric": "70B-shaped decode step ms/token (BASELINE config 5), 1 MI355X", "value": round(t_adakv, 3),
        "unit": "ms/token", "n_gpus": 1, "steps": steps, "warmup": warm, "higher_is_better": False,
        "dtype": "bf16", "data": "synthetic (random-init weights, random K/V cache)",
        "config": {"workload": "Llama-3-70B-shaped decode step via patch_model (BASELINE config 5)",
                   "layers": L, "batch": B, "context": S0, "n_q_heads": 64, "n_kv_heads": 8, "head_dim": 128,
                   "hidden": 8192, "block_size": 16, "avg_budget": 8, "cache": "StaticCache",
                   "parameters": n_params},
        "dense_hip_ms_per_token": round(t_dense_hip, 3), "dense_sdpa_ms_per_token": round(t_dense, 3),
        "noop_attention_ms_per_token": round(t_noop, 3),
        "attention_share_adakv": round(max(t_adakv - t_noop, 0.0) / t_adakv, 4),
        "attention_share_dense_hip": round(max(t_dense_hip - t_noop, 0.0) / t_dense_hip, 4),
        "attention_share_dense_sdpa": round(max(t_dense - t_noop, 0.0) / t_dense, 4),
        "adakv_attention_us_per_layer": round(max(t_adakv - t_noop, 0.0) * 1e3 / L, 2),
        "dense_hip_attention_us_per_layer": round(max(t_dense_hip - t_noop, 0.0) * 1e3 / L, 2),
        "speedup_vs_dense_hip_step": round(t_dense_hip / t_adakv, 3),
        "speedup_vs_dense_sdpa_step": round(t_dense / t_adakv, 3),
    }
    del model, cache
    torch.cuda.empty_cache()
    return res


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one MI355X; multi-GPU runs are not part of it "
              "(see DESIGN.md for how the path would shard)", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import torch

    from adakv_amd import _capi, ops
    _capi.load()
    assert torch.cuda.is_available(), "bench.py needs a ROCm device"
    if args.model_step:
        print(json.dumps(model_step(args)), flush=True)
        return
    log(f"device {torch.cuda.get_device_name(0)}; building {args.layers} layers at ctx {args.ctx}")
    w = Workload(torch, ops, args.ctx, args.layers, args.avg_budget, args.seed)
    L = w.L
    steps, warmup = max(1, args.steps), max(0, args.warmup)
    # the other legs keep one graph per pass over the layers
    replays = max(1, math.ceil(steps / L))
    warm = max(1, math.ceil(warmup / L))
    cell_steps = replays * L
    stream = torch.cuda.Stream()

    log(f"timing {steps} layer-steps after {warmup} untimed ones")
    ms, wall = time_exact(torch, w.step, steps, warmup, L, stream)
    us_layer = ms * 1e3 / steps
    log(f"adakv fused: {us_layer:.2f} us/layer (events), wall {wall * 1e3 / steps:.2f} us/layer")

    nbytes = selection_bytes(torch, ops, w)
    gbps = nbytes["total"] / (us_layer * 1e-6) / 1e9

    # the step's two launches: the scan launch alone, exactly as the step
    # issues it (append + scores + softmax records), the same number of
    # times over the same layers; the select + decode launch is the rest
    ms_sc, _ = time_exact(torch, w.scan, steps, warmup, L, stream)
    us_sc = ms_sc * 1e3 / steps
    sc_bytes = scan_bytes(w)
    sc_gbps = sc_bytes["total"] / (us_sc * 1e-6) / 1e9
    log(f"scan launch: {us_sc:.2f} us/launch, {sc_gbps:.0f} GB/s")
    us_sd = max(us_layer - us_sc, 1e-3)
    sbuf = torch.zeros(1, w.Hq, w.c[0].shape[2], device="cuda", dtype=torch.float32)   # the minmax scan leg's scores
    sd_bytes = nbytes["kv"] + nbytes["q"] + nbytes["out"] + nbytes["meta"] + sc_bytes["records"]
    sd_gbps = sd_bytes / (us_sd * 1e-6) / 1e9
    log(f"select + decode launch (step - scan): {us_sd:.2f} us, {sd_gbps:.0f} GB/s")

    copy_gbps = stream_copy_gbps(torch)
    log(f"stream copy: {copy_gbps:.0f} GB/s")
    traffic = profiled_traffic(os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                            "decode_step_kernels_128k_pmc.md"))

    dense_us = None
    if not args.no_dense:
        g_d = capture(torch, w.dense, L, stream)
        ms_d, _ = time_graph(torch, g_d, max(1, replays // 8), 1)
        dense_us = ms_d * 1e3 / (max(1, replays // 8) * L)
        dense_gbps = (2 * w.Hkv * w.S * w.D * 2) / (dense_us * 1e-6) / 1e9
        log(f"dense flash-decode: {dense_us:.1f} us/layer ({dense_gbps:.0f} GB/s)")

    cells = None
    if not args.no_cells:
        w.build_cells(args.avg_budget)
        cells = {"adakv": {"us_per_layer": round(us_layer, 3), "estimator": "centroid",
                           "budget_policy": "adaptive",
                           "summary_bytes_per_layer": int(w.c[0][:, :, : w.nb].numel() * 2)}}
        for name, fn, est, pol in (("quest", w.quest, "minmax", "fixed"),
                                   ("adakv_cf", w.adakv_cf, "centroid", "fixed"),
                                   ("adakv_nucleus", w.adakv_nucleus, "centroid", "adaptive_nucleus"),
                                   ("streaming", w.streaming, None, "fixed")):
            g_c = capture(torch, fn, L, stream)
            ms_c, _ = time_graph(torch, g_c, replays, warm)
            us_c = ms_c * 1e3 / cell_steps
            summ = w.m[0] if est == "minmax" else w.c[0] if est == "centroid" else None
            cells[name] = {"us_per_layer": round(us_c, 3), "estimator": est, "budget_policy": pol,
                           "summary_bytes_per_layer": 0 if summ is None else int(summ[:, :, : w.nb].numel() * 2)}
            log(f"{name}: {us_c:.2f} us/layer")
            del g_c
        g_ms = capture(torch, lambda l: w.minmax_scores(l, sbuf), L, stream)
        ms_ms, _ = time_graph(torch, g_ms, replays, warm)
        us_ms = ms_ms * 1e3 / cell_steps
        ms_bytes = 2 * nbytes["centroid"] + nbytes["q"] + w.Hq * w.nb * 4
        cells["quest"]["scan_us"] = round(us_ms, 3)
        cells["quest"]["scan_GBps"] = round(ms_bytes / (us_ms * 1e-6) / 1e9, 1)
        log(f"minmax scan: {us_ms:.2f} us/launch, {ms_bytes / (us_ms * 1e-6) / 1e9:.0f} GB/s")
        del g_ms
        if dense_us is not None:
            cells["dense"] = {"us_per_layer": round(dense_us, 2), "estimator": None,
                              "budget_policy": None, "summary_bytes_per_layer": 0}

    avg32 = None
    if not args.no_cells and args.avg_budget != 32:
        # BASELINE config 3's second budget on the same layers: avg_budget 32
        # (about 27 content blocks per head, so every needle fits)
        b8 = w.budget
        w.budget = ops.BudgetParams(avg_budget=32)
        g32 = capture(torch, w.step, L, stream)
        ms32, _ = time_graph(torch, g32, replays, warm)
        us32 = ms32 * 1e3 / cell_steps
        nb32 = selection_bytes(torch, ops, w)
        w.budget = b8
        avg32 = {"avg_budget": 32, "us_per_layer": round(us32, 3), "bytes_per_layer": int(nb32["total"]),
                 "kv_bytes_per_layer": int(nb32["kv"]),
                 "union_blocks_per_layer": round(nb32["union_blocks_per_layer"], 2),
                 "achieved_GBps": round(nb32["total"] / (us32 * 1e-6) / 1e9, 1)}
        log(f"adakv fused, avg_budget 32: {us32:.2f} us/layer")
        del g32

    sweep = None
    if not args.no_sweep:
        # latency against context (the reference's efficiency experiment,
        # bench_decode_latency.py:1-24): the same layer shape, 8 rotated layers
        # per context, AdaKV step and dense decode
        sweep = []
        for ctx in [int(x) for x in args.sweep_ctx.split(",") if x]:
            ws = Workload(torch, ops, ctx, 8, args.avg_budget, args.seed + 1)
            g1 = capture(torch, ws.step, ws.L, stream)
            ms1, _ = time_graph(torch, g1, 16, 2)
            g2 = capture(torch, ws.dense, ws.L, stream)
            ms2, _ = time_graph(torch, g2, 4, 1)
            a_us, d_us = ms1 * 1e3 / (16 * ws.L), ms2 * 1e3 / (4 * ws.L)
            sweep.append({"context": ctx, "adakv_us_per_layer": round(a_us, 2),
                          "dense_us_per_layer": round(d_us, 2), "speedup": round(d_us / a_us, 2),
                          # the fused select + decode kernel serves up to 16384 blocks (512 threads x 32)
                          "path": "fused (2 launches)" if ws.nb <= 16384 else "plan + decode (3 launches)"})
            log(f"ctx {ctx}: adakv {a_us:.2f} us/layer, dense {d_us:.2f} us/layer")
            del g1, g2, ws
            torch.cuda.empty_cache()

    ragged = None
    if not args.no_ragged:
        ragged = ragged_batch(torch, ops, stream, args.seed + 2)

    evict = None
    if not args.no_evict:
        evict = evict_bench(torch, ops, w, stream, args.seed + 3, args.h2o_len)

    cpu = None
    if not args.no_cpu:
        sec, runs = cpu_baseline(torch, w, args.cpu_seconds)
        cpu = {"value": round(sec * 1e6, 1), "unit": "us/layer", "cores": 1, "kind": "port",
               "sample": f"oracle.sparse_attention on layer 0 of this workload (ctx {w.S}, "
                         f"32/8 heads, fp32 NumPy, GQA-expanded K/V), {runs} runs, median of "
                         f"runs after the first; host has {os.cpu_count()} CPUs, "
                         f"{len(os.sched_getaffinity(0))} in affinity, NumPy einsum single-threaded"}
        log(f"cpu oracle: {sec:.2f} s/layer")

    res = {
        "metric": METRIC, "value": round(us_layer, 3), "unit": "us/layer", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(us_layer / 1e3, 6),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "llama3.1-8b attention layer decode, ctx 131072, avg_budget 8 (BASELINE config 3)",
                   "batch": 1, "n_q_heads": w.Hq, "n_kv_heads": w.Hkv, "head_dim": w.D,
                   "context": w.S, "block_size": w.BS, "avg_budget": args.avg_budget,
                   "layers_rotated": L},
        "achieved_GBps": round(gbps, 1),
        "bytes_per_layer": int(nbytes["total"]),
        "kv_bytes_per_layer": int(nbytes["kv"]),
        "union_blocks_per_layer": round(nbytes["union_blocks_per_layer"], 2),
        "roofline_frac_whole_op": round(gbps / PEAK_HBM_GBPS, 4),
        "dense_us_per_layer": None if dense_us is None else round(dense_us, 2),
        "speedup_vs_dense": None if dense_us is None else round(dense_us / us_layer, 2),
        "stream_copy_GBps": round(copy_gbps, 1),
        "roofline": {"kernel": "score_kernel (the step's scan launch: append + scores + records)",
                     "bound": "hbm", "achieved": round(sc_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(sc_gbps / PEAK_HBM_GBPS, 4),
                     "traffic": traffic.get("score_kernel") if (traffic and args.ctx == 131072 and L == 32) else None,
                     "launch_us": round(us_sc, 3), "bytes_per_launch": int(sc_bytes["total"]),
                     "bytes": {k: int(v) for k, v in sc_bytes.items()},
                     "frac_of_stream_copy": round(sc_gbps / copy_gbps, 4)},
        "roofline_select_decode": {"kernel": "select_decode_kernel (budget + selection + decode), timed as "
                                             "the step minus the scan launch (includes the launch gap)",
                                   "bound": "hbm", "achieved": round(sd_gbps, 1), "peak": PEAK_HBM_GBPS,
                                   "unit": "GB/s", "frac": round(sd_gbps / PEAK_HBM_GBPS, 4),
                                   "traffic": traffic.get("select_decode_kernel") if (
                                       traffic and args.ctx == 131072 and L == 32) else None,
                                   "launch_us": round(us_sd, 3), "bytes_per_launch": int(sd_bytes)},
        "cpu_baseline": cpu,
        "cells": cells,
        "avg_budget_32": avg32,
        "ctx_sweep": sweep,
        "ragged_batch": ragged,
        "eviction": evict,
        "model_step": None,
    }
    if not args.no_model_step:
        # BASELINE config 5 (80-layer, 70B-shaped model through patch_model),
        # after the layer workload's memory is released: its weights and cache
        # take 211 GiB
        del w
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        res["model_step"] = model_step(args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
