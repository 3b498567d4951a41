"""The HuggingFace hook's decode steps, checked where the hook launches them
(adakv/patch.py:90-121 is the reference's hook).

``HookCheck`` wraps ``adakv_amd.ops.decode_fused`` -- which ``adakv.patch``
calls once per layer and decode step -- so that it also returns the
selection, and checks every call, sequence by sequence, before the model
goes on:

* the summaries the hook passes (kept across steps, refreshed by append_new,
  permuted by beam reordering) equal a fresh ``centroid_build`` of the live
  tokens of that sequence;
* the selection equals the oracle's budget and selection (adakv/budget.py,
  adakv/selector.py) on those summaries, near-ties excluded and counted
  (``compare_selection``);
* the output equals fp64 attention over the GPU's own selection.

Only the centroid estimator is checked (minmax summaries are not rebuilt here).
"""
from __future__ import annotations

import math

import numpy as np

from gpu_util import BF16_ATOL, REL_L2, O, compare_selection, rel_l2, torch


class HookCheck:
    def __init__(self):
        self.calls = 0          # decode_fused calls checked (one per layer and step, or per sequence)
        self.sequences = 0      # (call, sequence) pairs checked
        self.heads = 0          # q-heads whose selection was compared
        self.excluded = 0       # of those, excluded as near-ties
        self.appends = 0        # calls that refreshed the summaries incrementally (append_new > 0)

    def __enter__(self):
        from adakv_amd import ops
        self.ops, self.real = ops, ops.decode_fused
        ops.decode_fused = self._wrapped
        return self

    def __exit__(self, *exc):
        self.ops.decode_fused = self.real
        return False

    def _wrapped(self, q, k, v, centroid, block_size, budget, seq_lens=None, append_new=0, sm_scale=None,
                 out=None, return_selection=False, estimator=None):
        res = self.real(q, k, v, centroid, block_size, budget, seq_lens=seq_lens, append_new=append_new,
                        sm_scale=sm_scale, out=out, return_selection=True, estimator=estimator)
        if estimator in (None, "centroid"):
            self._check(q, k, v, centroid, block_size, budget, seq_lens, sm_scale, append_new, *res)
        return res if return_selection else res[0]

    def _check(self, q, k, v, centroid, bs, budget, seq_lens, sm_scale, append_new, out, table, lens):
        torch.cuda.synchronize()
        B, Hq, D = q.shape
        Hkv, S = k.shape[1], k.shape[2]
        G = Hq // Hkv
        L_b = [S] * B if seq_lens is None else [int(x) for x in seq_lens.tolist()]
        scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
        t, n, o = table.cpu().numpy(), lens.cpu().numpy(), out.float().cpu().numpy()
        self.calls += 1
        self.appends += int(append_new > 0)
        for b in range(B):
            L = L_b[b]
            nb = -(-L // bs)
            if nb == 0:
                continue
            fresh = self.ops.centroid_build(k[b:b + 1, :, :L], bs, centroid_dtype=centroid.dtype)
            torch.cuda.synchronize()
            assert torch.equal(centroid[b:b + 1, :, :nb], fresh[:, :, :nb]), \
                f"sequence {b}: the hook's summaries differ from a rebuild of its {L} tokens"
            cent = centroid[b, :, :nb].float().cpu().numpy()
            q_np = q[b].float().cpu().numpy()
            scores = O.block_scores(q_np, {"kind": "centroid", "centroid": O.expand_gqa(cent, Hq)})
            lo, hi, target, _ = O.budget_bounds(nb, budget.avg_budget, budget.k_min, budget.k_max,
                                                budget.n_sink_blocks, budget.n_local_blocks, budget.c_min)
            floor = min(budget.n_sink_blocks, nb) + min(budget.n_local_blocks, nb) + budget.c_min
            k_or = O.allocate_budget(scores, budget.avg_budget, min(budget.k_min, nb), min(budget.k_max, nb),
                                     temperature=budget.temperature, policy=budget.budget_policy,
                                     nucleus_p=budget.nucleus_p, floor=floor)
            w_or = O.budget_weights(scores, "adaptive" if budget.budget_policy == "fixed" else budget.budget_policy,
                                    budget.temperature, budget.nucleus_p)
            self.excluded += compare_selection(scores, t[b], n[b], k_oracle=k_or, w_oracle=w_or, lo=lo,
                                               target=target, sink=budget.n_sink_blocks,
                                               local=budget.n_local_blocks, cmin=budget.c_min,
                                               policy=budget.budget_policy)
            self.heads += Hq
            self.sequences += 1
            ref = np.zeros((Hq, D), np.float64)
            for h in range(Hq):
                blocks = sorted({int(x) for x in t[b, h, : int(n[b, h])] if 0 <= int(x) < nb})
                idx = torch.from_numpy(np.concatenate(
                    [np.arange(x * bs, min((x + 1) * bs, L)) for x in blocks])).to(k.device)
                kk = k[b, h // G].index_select(0, idx).double().cpu().numpy()
                vv = v[b, h // G].index_select(0, idx).double().cpu().numpy()
                lg = kk @ q_np[h].astype(np.float64) * scale
                p = np.exp(lg - lg.max())
                ref[h] = p @ vv / p.sum()
            err = float(np.abs(o[b] - ref).max())
            assert err <= BF16_ATOL and rel_l2(o[b], ref) < REL_L2, \
                f"sequence {b}: output max abs {err:.2e} against fp64 over the GPU's selection"
