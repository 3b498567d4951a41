"""adakv_decode_fused_noalloc, the allocation-free variant of adakv_decode_fused,
through the C ABI on the GPU.

The variant takes no workspace: its scratch is a static device array inside
the library, shared by every call on the GPU.  On calls in a row -- the second
one smaller than the first, then the three-launch paths (fp32 K/V, whose
split-K merge uses the hand-off counters at the front of the scratch, and the
nucleus budget) and the first geometry again -- its output, table rows and
counts and appended centroids equal adakv_decode_fused's on the same inputs
bit for bit, and its output within the bf16 bar (both run the same kernels;
only the scratch differs).  (The refusal of a geometry whose
workspace exceeds the array is a host check, tested on the CPU.)
"""
from __future__ import annotations

import ctypes
import math

import pytest

from gpu_util import DEV, need_gpu, say, torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    need_gpu()


def _ops():
    from adakv_amd import ops
    return ops


def _noalloc(q, k, v, c, bs, budget, seq_lens=None, append_new=0):
    """ops.decode_fused's argument marshalling, calling the no-alloc entry point."""
    from adakv_amd import _capi as C
    ops = _ops()
    B, Hq, D = q.shape
    _, Hkv, S, _ = k.shape
    g = ops.geometry(B, Hq, Hkv, D, bs, S, c.shape[2])
    cb = budget.to_c()
    T = C.load().adakv_table_width(ctypes.byref(g), ctypes.byref(cb))
    out = torch.empty(B, Hq, D, dtype=q.dtype, device=q.device)
    table = torch.empty(B, Hq, T, dtype=torch.int32, device=q.device)
    lens = torch.empty(B, Hq, dtype=torch.int32, device=q.device)
    sel = C.Selection(table.data_ptr(), T, lens.data_ptr())
    st = C.load().adakv_decode_fused_noalloc(
        ctypes.byref(g), ctypes.byref(ops._q(q)), ctypes.byref(ops._kv(k, v)),
        ctypes.byref(ops._centroid(c, D)), ops._ptr(seq_lens), ctypes.byref(cb), ctypes.byref(sel),
        int(append_new), ctypes.c_float(1.0 / math.sqrt(D)), ctypes.byref(ops._out(out)),
        ops._stream(q.device))
    C.check(st, "decode_fused_noalloc")
    return out, table, lens


def _case(seed, B, Hq, Hkv, D, S, dt, lens=None, policy="adaptive", avg=8):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(B, Hq, D, device=DEV, dtype=dt, generator=gen)
    k = torch.randn(B, Hkv, S, D, device=DEV, dtype=dt, generator=gen)
    v = torch.randn(B, Hkv, S, D, device=DEV, dtype=dt, generator=gen)
    k[:, : Hkv // 2] *= 3.0                       # peaked and flat heads: counts differ per head
    sl = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=DEV)
    c = _ops().centroid_build(k, 16, seq_lens=sl)
    budget = _ops().BudgetParams(avg_budget=avg, budget_policy=policy)
    return q, k, v, c, sl, budget


def _check(name, q, k, v, c, sl, budget):
    ops = _ops()
    c_ref, c_new = c.clone(), c.clone()
    ref, t_ref, n_ref = ops.decode_fused(q, k, v, c_ref, 16, budget, seq_lens=sl, append_new=1,
                                         return_selection=True)
    got, t_got, n_got = _noalloc(q, k, v, c_new, 16, budget, seq_lens=sl, append_new=1)
    torch.cuda.synchronize()
    assert torch.equal(n_got, n_ref), name
    for b in range(q.shape[0]):
        for h in range(q.shape[1]):
            n = int(n_ref[b, h])
            assert torch.equal(t_got[b, h, :n], t_ref[b, h, :n]), (name, b, h)
    # Same blocks, same kernels: the outputs differ at most by the order in which
    # the decode waves took the tiles (a candidate's wave follows its slot in an
    # LDS compaction), i.e. by fp32 summation order before the final rounding.
    err = float((got.float() - ref.float()).abs().max())
    tol = 1e-5 if got.dtype == torch.float32 else 1e-2
    assert err <= tol, (name, err)
    assert torch.equal(c_new, c_ref), name          # the appended centroids bit for bit
    say(f"{name}: {int(n_ref.sum())} selected blocks and centroids bit-identical, output max|diff| {err:.1e}")


def test_noalloc_equals_fused_on_calls_in_a_row():
    say("no-alloc: call 1, batch 2 ragged (65536, 40001 tokens), 32 q / 8 KV heads, bf16")
    _check("call 1", *_case(0, 2, 32, 8, 128, 65536, torch.bfloat16, lens=[65536, 40001]))
    say("no-alloc: call 2 (smaller), batch 1, 16 q / 4 KV heads, head_dim 64, 3000 tokens, fp16")
    _check("call 2", *_case(1, 1, 16, 4, 64, 3000, torch.float16))
    say("no-alloc: call 3, fp32 K/V (score, select, split-K decode with counters), 2048 tokens")
    _check("call 3", *_case(2, 1, 8, 2, 128, 2048, torch.float32))
    say("no-alloc: call 4, nucleus budget (score, nucleus, select-decode), 8192 tokens")
    _check("call 4", *_case(3, 1, 32, 8, 128, 8192, torch.bfloat16, policy="adaptive_nucleus"))
    say("no-alloc: call 5, call 1's geometry again")
    _check("call 5", *_case(4, 2, 32, 8, 128, 65536, torch.bfloat16, lens=[1000, 65536]))

