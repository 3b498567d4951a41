"""The BASELINE configurations at full size on the GPU, through the C ABI.

* config 2: Llama-3.1-8B layer at context 32768, half the KV heads peaked
  (keys scaled x4), avg_budget 8;
* config 3: context 131072 (and 262144) with 4 planted needle blocks per KV head (keys of
  needle j of KV head g = 3 * q[g * G + j] + noise), avg_budget 8 and 32;
* config 4: ragged batch of 8 sequences, lengths uniform in [16K, 128K], half
  the heads peaked, avg_budget 16.

At these sizes the oracle cannot replay the whole step cheaply, so each test
checks what the sizes allow: the selection is compared bit-exactly (near-ties
excluded and counted) with the oracle's budget and selection run on the GPU's
own centroids (fp32, the exact-parity mode, and bf16), each q-head must find
its own needle, and the output must match an fp64 attention over the GPU's own
selection (gathered block by block), within the bf16 tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import BF16_ATOL, DEV, REL_L2, compare_selection, need_gpu, rel_l2, say, torch
from oracle import adakv_oracle as O

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 32, 8, 128, 16
G = HQ // HKV
DEFAULTS = dict(kmin=2, kmax=64, sink=1, local=4, cmin=1)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    need_gpu()


def _ops():
    from adakv_amd import ops
    return ops


def _oracle_check(q_np, cent_kv, table, lens, avg):
    """Oracle budget + selection on the GPU's centroids [Hkv, nb, D]; compare."""
    p = DEFAULTS
    nb = cent_kv.shape[1]
    cent = O.expand_gqa(cent_kv.astype(np.float32), HQ)
    scores = O.block_scores(q_np, {"kind": "centroid", "centroid": cent})
    lo, hi, target, _ = O.budget_bounds(nb, avg, p["kmin"], p["kmax"], p["sink"], p["local"], p["cmin"])
    k = O.allocate_budget(scores, avg, min(p["kmin"], nb), min(p["kmax"], nb),
                          floor=min(p["sink"], nb) + min(p["local"], nb) + p["cmin"])
    w = O.budget_weights(scores)
    excl = compare_selection(scores, table, lens, k_oracle=k, w_oracle=w, lo=lo, target=target,
                             sink=p["sink"], local=p["local"], cmin=p["cmin"], policy="adaptive")
    say(f"  selection parity: {HQ - excl}/{HQ} heads compared, {excl} excluded as near-ties")
    return k


def _ref_selected(q, k, v, table, lens, length):
    """fp64 attention of every q-head over its own selected blocks (duplicates
    once), gathering only those rows from the device tensors [Hkv, S, D]."""
    out = np.zeros((HQ, D), np.float64)
    nb = -(-length // BS)
    for h in range(HQ):
        blocks = sorted({int(b) for b in table[h, : int(lens[h])] if 0 <= int(b) < nb})
        idx = np.concatenate([np.arange(b * BS, min((b + 1) * BS, length)) for b in blocks])
        it = torch.from_numpy(idx).to(DEV)
        kk = k[h // G].index_select(0, it).double().cpu().numpy()
        vv = v[h // G].index_select(0, it).double().cpu().numpy()
        lg = kk @ q[h].astype(np.float64) / np.sqrt(D)
        p = np.exp(lg - lg.max())
        out[h] = p @ vv / p.sum()
    return out


def _check_output(got, ref):
    err = float(np.abs(got - ref).max())
    r = rel_l2(got, ref)
    say(f"  output: max abs {err:.2e}, rel L2 {r:.2e}")
    assert err <= BF16_ATOL and r < REL_L2


def _needle_layer(S, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(1, HQ, D, device=DEV, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, HKV, S, D, device=DEV, generator=gen).to(torch.bfloat16)
    v = torch.randn(1, HKV, S, D, device=DEV, generator=gen).to(torch.bfloat16)
    nb = -(-S // BS)
    rng = np.random.RandomState(seed)
    pos = np.stack([rng.choice(np.arange(1, nb - 4), 4, replace=False) for _ in range(HKV)])
    for g in range(HKV):
        for j in range(4):
            b = int(pos[g, j])
            noise = torch.randn(BS, D, device=DEV, generator=gen)
            k[0, g, b * BS:(b + 1) * BS] = (3.0 * q[0, g * G + j].float()[None] + noise).to(torch.bfloat16)
    return q, k, v, pos


@pytest.mark.parametrize("avg", [8, 32])
@pytest.mark.parametrize("cdt", [torch.float32, torch.bfloat16])
def test_config3_needles_128k(avg, cdt):
    ops = _ops()
    S = 131072
    say(f"config 3: ctx {S}, needles, avg_budget {avg}, centroids {cdt}")
    q, k, v, pos = _needle_layer(S, seed=7)
    c = ops.centroid_build(k, BS, centroid_dtype=cdt)
    out, table, lens = ops.decode_fused(q, k, v, c, BS, ops.BudgetParams(avg_budget=avg),
                                        append_new=1, return_selection=True)
    torch.cuda.synchronize()
    table, lens = table[0].cpu().numpy(), lens[0].cpu().numpy()
    q_np = q[0].float().cpu().numpy()
    _oracle_check(q_np, c[0].float().cpu().numpy(), table, lens, avg)
    # every q-head finds its own needle
    for g in range(HKV):
        for j in range(4):
            h = g * G + j
            assert int(pos[g, j]) in set(table[h, : lens[h]].tolist()), f"head {h} missed its needle"
    assert abs(lens.mean() - avg) <= 1.0
    _check_output(out[0].float().cpu().numpy(), _ref_selected(q_np, k[0], v[0], table, lens, S))


@pytest.mark.parametrize("S", [65536, 100000])
def test_needles_two_tiles_per_wave(S):
    """4096 and 6250 blocks per KV head: the matrix-core scan runs 2 tiles per
    wave (4 from 7937 blocks on, 1 below 3969, at 8 KV heads and batch 1), so
    its records cover 128 rows."""
    ops = _ops()
    avg = 8
    say(f"needles: ctx {S}, avg_budget {avg}, bf16 centroids (scan at 2 tiles per wave)")
    q, k, v, pos = _needle_layer(S, seed=11)
    c = ops.centroid_build(k, BS, centroid_dtype=torch.bfloat16)
    out, table, lens = ops.decode_fused(q, k, v, c, BS, ops.BudgetParams(avg_budget=avg),
                                        append_new=1, return_selection=True)
    torch.cuda.synchronize()
    table, lens = table[0].cpu().numpy(), lens[0].cpu().numpy()
    q_np = q[0].float().cpu().numpy()
    _oracle_check(q_np, c[0].float().cpu().numpy(), table, lens, avg)
    assert abs(lens.mean() - avg) <= 1.0
    _check_output(out[0].float().cpu().numpy(), _ref_selected(q_np, k[0], v[0], table, lens, S))


@pytest.mark.parametrize("cdt", [torch.float32, torch.bfloat16])
def test_needles_256k(cdt):
    """Context 262,144 (16,384 blocks per KV head): the selection runs at its
    widest shape (512 threads, 32 blocks per thread), the matrix-core scan
    (bf16 centroids) at 4 tiles per wave; every q-head finds its own needle."""
    ops = _ops()
    S, avg = 262144, 8
    say(f"needles: ctx {S}, avg_budget {avg}, centroids {cdt}")
    q, k, v, pos = _needle_layer(S, seed=13)
    c = ops.centroid_build(k, BS, centroid_dtype=cdt)
    out, table, lens = ops.decode_fused(q, k, v, c, BS, ops.BudgetParams(avg_budget=avg),
                                        append_new=1, return_selection=True)
    torch.cuda.synchronize()
    table, lens = table[0].cpu().numpy(), lens[0].cpu().numpy()
    q_np = q[0].float().cpu().numpy()
    _oracle_check(q_np, c[0].float().cpu().numpy(), table, lens, avg)
    for g in range(HKV):
        for j in range(4):
            h = g * G + j
            assert int(pos[g, j]) in set(table[h, : lens[h]].tolist()), f"head {h} missed its needle"
    assert abs(lens.mean() - avg) <= 1.0
    _check_output(out[0].float().cpu().numpy(), _ref_selected(q_np, k[0], v[0], table, lens, S))


def test_config2_32k_half_peaked():
    ops = _ops()
    S, avg = 32768, 8
    say(f"config 2: ctx {S}, half the KV heads peaked (keys x4), avg_budget {avg}")
    gen = torch.Generator(device=DEV).manual_seed(2)
    q = torch.randn(1, HQ, D, device=DEV, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, HKV, S, D, device=DEV, generator=gen)
    k[:, : HKV // 2] *= 4.0
    k = k.to(torch.bfloat16)
    v = torch.randn(1, HKV, S, D, device=DEV, generator=gen).to(torch.bfloat16)
    c = ops.centroid_build(k, BS, centroid_dtype=torch.float32)
    out, table, lens = ops.decode_fused(q, k, v, c, BS, ops.BudgetParams(avg_budget=avg),
                                        return_selection=True)
    torch.cuda.synchronize()
    table, lens = table[0].cpu().numpy(), lens[0].cpu().numpy()
    q_np = q[0].float().cpu().numpy()
    _oracle_check(q_np, c[0].float().cpu().numpy(), table, lens, avg)
    # peaked heads (low entropy) receive fewer blocks than flat heads (test_reference.py:88-100)
    assert lens[: HQ // 2].mean() < lens[HQ // 2:].mean()
    _check_output(out[0].float().cpu().numpy(), _ref_selected(q_np, k[0], v[0], table, lens, S))


@pytest.mark.parametrize("cdt", [torch.float32, torch.bfloat16])
def test_config4_ragged_batch(cdt):
    ops = _ops()
    B, avg = 8, 16
    rng = np.random.RandomState(4)
    lens_tok = rng.randint(16384, 131072 + 1, size=B).astype(np.int32)
    S = int(lens_tok.max())
    say(f"config 4: ragged batch of {B}, lengths {lens_tok.tolist()}, avg_budget {avg}, centroids {cdt}")
    gen = torch.Generator(device=DEV).manual_seed(4)
    q = torch.randn(B, HQ, D, device=DEV, generator=gen).to(torch.bfloat16)
    k = torch.empty(B, HKV, S, D, device=DEV, dtype=torch.bfloat16)
    v = torch.empty(B, HKV, S, D, device=DEV, dtype=torch.bfloat16)
    for b in range(B):
        kb = torch.randn(HKV, S, D, device=DEV, generator=gen)
        kb[: HKV // 2] *= 4.0          # half the heads peaked
        k[b] = kb.to(torch.bfloat16)
        v[b] = torch.randn(HKV, S, D, device=DEV, generator=gen).to(torch.bfloat16)
    sl = torch.from_numpy(lens_tok).to(DEV)
    c = ops.centroid_build(k, BS, seq_lens=sl, centroid_dtype=cdt)
    out, table, lens = ops.decode_fused(q, k, v, c, BS, ops.BudgetParams(avg_budget=avg), seq_lens=sl,
                                        return_selection=True)
    torch.cuda.synchronize()
    table, lens = table.cpu().numpy(), lens.cpu().numpy()
    for b in range(B):
        Sb = int(lens_tok[b])
        nb = -(-Sb // BS)
        say(f"  sequence {b}: {Sb} tokens, {nb} blocks")
        q_np = q[b].float().cpu().numpy()
        _oracle_check(q_np, c[b, :, :nb].float().cpu().numpy(), table[b], lens[b], avg)
        _check_output(out[b].float().cpu().numpy(), _ref_selected(q_np, k[b], v[b], table[b], lens[b], Sb))


@pytest.mark.parametrize("cap", [131072, 262144])
@pytest.mark.parametrize("cdt", [torch.float32, torch.bfloat16])
def test_overallocated_summaries_match_tight(cdt, cap):
    """A summary buffer allocated for 128K / 256K tokens while K holds 20000:
    the scan and the selection kernels are shaped by the length bound (not the
    buffer; a 16384-block buffer stays on the fused path), so the step's
    selection and output are bit-identical to those over a tight buffer."""
    ops = _ops()
    S, avg = 20000, 8
    say(f"over-allocated summaries: ctx {S} in a buffer of {cap // BS} blocks, centroids {cdt}")
    q, k, v, _ = _needle_layer(S, seed=13)
    tight = ops.centroid_build(k, BS, centroid_dtype=cdt)
    wide = ops.centroid_build(k, BS, centroid_dtype=cdt, max_blocks=cap // BS)
    assert wide.shape[2] == cap // BS and tight.shape[2] == -(-S // BS)
    p = ops.BudgetParams(avg_budget=avg)
    o1, t1, l1 = ops.decode_fused(q, k, v, tight, BS, p, return_selection=True)
    o2, t2, l2 = ops.decode_fused(q, k, v, wide, BS, p, return_selection=True)
    torch.cuda.synchronize()
    assert torch.equal(l1, l2)
    w = t1.shape[2]
    assert torch.equal(t1, t2[..., :w]) and bool((t2[..., w:] == -1).all())
    assert torch.equal(o1, o2)
