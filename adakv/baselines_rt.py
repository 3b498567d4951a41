"""H2O / SnapKV eviction baselines on the HIP path (adakv/baselines_rt.py).

Both baselines pick, once at prefill, which KV blocks a sequence keeps, from
the prompt's own attention, and attend that frozen set (plus the current sink
and local blocks) at every decode step.  The functions keep the reference's
names, arguments and per-query-head semantics; the work runs in
libadakv_amd.so:

* key importance (``adakv_key_importance``): per query head, the attention
  each key receives summed over the causal prompt queries (H2O) or over the
  last ``obs_window`` queries (SnapKV), streamed through the matrix cores in
  two passes (row log-sum-exp, then column sums) -- nothing of size
  [H, L, L] or [H, chunk, L] is formed, and a KV head serves its query heads
  without being expanded;
* SnapKV's max pool (``adakv_importance_pool``);
* the retained set (``adakv_retain_blocks``): block sums, forced sink and
  local blocks, top content blocks;
* tables (``adakv_frozen_table``, ``adakv_mask_table``).

Inputs are CUDA (ROCm) tensors; there is no CPU path (the NumPy oracle under
``oracle/`` is the CPU reference, for tests).
"""
from __future__ import annotations

import ctypes
import math

import torch

from adakv_amd import _capi as C
from adakv_amd.ops import _dt, _on_device, _ptr, _stream

__all__ = [
    "expand_kv_heads",
    "key_importance",
    "h2o_key_importance_torch",
    "snapkv_key_importance_torch",
    "importance_pool",
    "retain_blocks_torch",
    "retain_blocks_table",
    "h2o_retained_mask_torch",
    "snapkv_retained_mask_torch",
    "mask_to_block_table",
    "frozen_decode_block_table",
    "frozen_table",
]


def expand_kv_heads(x: torch.Tensor, group: int) -> torch.Tensor:
    """[Hkv, L, D] -> [Hq, L, D] by repeating each KV head ``group`` times
    (adakv/baselines_rt.py:38-40).  The kernels below never need it: they map
    query head h to KV head h // group themselves."""
    return x.repeat_interleave(group, dim=0) if group > 1 else x


def _prompt(Q: torch.Tensor, K: torch.Tensor) -> C.Prompt:
    if Q.dim() != 3 or K.dim() != 3:
        raise ValueError(f"Q and K must be [H, L, D], got {tuple(Q.shape)} and {tuple(K.shape)}")
    Hq, L, D = Q.shape
    Hkv = K.shape[0]
    if K.shape[1:] != (L, D) or Hq % Hkv:
        raise ValueError(f"Q {tuple(Q.shape)} and K {tuple(K.shape)}: K must be [Hkv, L, D] with Hkv | Hq")
    if Q.dtype != K.dtype:
        raise ValueError("Q and K must share one dtype")
    if Q.stride(-1) != 1 or K.stride(-1) != 1:
        raise ValueError("head_dim must be the contiguous axis of Q and K")
    return C.Prompt(Q.data_ptr(), K.data_ptr(), _dt(Q), Hq, Hkv, D, L,
                    Q.stride(0), Q.stride(1), K.stride(0), K.stride(1))


def key_importance(Q: torch.Tensor, K: torch.Tensor, first_query: int = 0, sm_scale=None) -> torch.Tensor:
    """[Hq, L] fp32: the attention each key receives, summed over the queries
    at positions [first_query, L) that can see it (adakv/baselines.py:63-79
    for first_query 0, 101-114 for a window).  Q [Hq, L, D], K [Hkv, L, D]
    (or already expanded to Hq heads); sm_scale defaults to 1/sqrt(D)."""
    dev = _on_device(Q, K)
    p = _prompt(Q, K)
    Hq, L, D = Q.shape
    sm_scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    lib = C.load()
    nbytes = lib.adakv_importance_workspace_bytes(ctypes.byref(p), int(first_query))
    if nbytes == 0:
        raise ValueError(f"key_importance: unsupported prompt (first_query={first_query}, L={L}, D={D})")
    imp = torch.empty(Hq, L, dtype=torch.float32, device=dev)
    lse = torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=dev)
    C.check(lib.adakv_key_importance(ctypes.byref(p), int(first_query), ctypes.c_float(sm_scale), _ptr(imp), L,
                                     _ptr(lse), nbytes, _stream(dev)), "key_importance")
    return imp


def h2o_key_importance_torch(Q: torch.Tensor, K: torch.Tensor, chunk: int = 256) -> torch.Tensor:
    """Accumulated causal attention of every key (adakv/baselines_rt.py:43-64).
    ``chunk`` is accepted for the reference's signature; the kernels stream
    queries 16 at a time and never hold a [H, chunk, L] block."""
    return key_importance(Q, K, 0)


def importance_pool(x: torch.Tensor, kernel: int) -> torch.Tensor:
    """Same-length max pool over the last axis, window clipped at the edges
    (SnapKV's max_pool1d, adakv/baselines_rt.py:79-80; adakv/baselines.py:82-92)."""
    dev = _on_device(x)
    if kernel <= 1:
        return x
    if kernel % 2 == 0:
        raise ValueError("pool_kernel must be odd (a same-length pool)")
    if x.dim() != 2 or x.dtype != torch.float32 or x.stride(-1) != 1:
        raise ValueError("importance must be [H, L] float32 with a contiguous last axis")
    H, L = x.shape
    out = torch.empty(H, x.stride(0), dtype=torch.float32, device=dev)[:, :L]
    C.check(C.load().adakv_importance_pool(_ptr(x), _ptr(out), H, L, x.stride(0), int(kernel), _stream(dev)),
            "importance_pool")
    return out


def snapkv_key_importance_torch(Q: torch.Tensor, K: torch.Tensor, obs_window: int = 32,
                                pool_kernel: int = 7) -> torch.Tensor:
    """SnapKV importance: the last ``obs_window`` queries, max-pooled over
    key positions (adakv/baselines_rt.py:67-80)."""
    L = Q.shape[1]
    w = int(min(obs_window, L))
    return importance_pool(key_importance(Q, K, L - w), pool_kernel)


def _retain(importance, block_size, n_real, budget, n_sink_blocks, n_local_blocks, c_min, with_table):
    dev = _on_device(importance)
    if importance.dim() != 2 or importance.dtype != torch.float32 or importance.stride(-1) != 1:
        raise ValueError("importance must be [H, L] float32 with a contiguous last axis")
    H, L = importance.shape
    n_real = int(n_real)
    if not 0 < n_real <= L:
        raise ValueError(f"n_real={n_real} outside (0, {L}]")
    bs = int(block_size)
    nb = -(-n_real // bs)
    sink, local = min(int(n_sink_blocks), nb), min(int(n_local_blocks), nb)
    k = min(max(int(budget), min(sink + local + int(c_min), nb)), nb)
    mask = torch.empty(H, nb, dtype=torch.uint8, device=dev)
    sel = table = lens = None
    if with_table:
        table = torch.empty(H, max(k, 1), dtype=torch.int32, device=dev)
        lens = torch.empty(H, dtype=torch.int32, device=dev)
        sel = C.Selection(table.data_ptr(), max(k, 1), lens.data_ptr())
    C.check(C.load().adakv_retain_blocks(_ptr(importance), H, importance.stride(0), n_real, bs, int(budget),
                                         int(n_sink_blocks), int(n_local_blocks), int(c_min), _ptr(mask), nb,
                                         ctypes.byref(sel) if sel is not None else None, _stream(dev)),
            "retain_blocks")
    return mask.view(torch.bool), (table[:, :k] if table is not None else None), lens


def retain_blocks_torch(importance: torch.Tensor, block_size: int, n_real: int, budget: int,
                        n_sink_blocks: int = 1, n_local_blocks: int = 4, c_min: int = 1) -> torch.Tensor:
    """Retained mask [H, nb] bool: k = clamp(budget, floor, nb) blocks per
    head -- sink, local, then the content blocks of largest importance sum
    (adakv/baselines_rt.py:83-127).  Equal sums: lower block first."""
    return _retain(importance, block_size, n_real, budget, n_sink_blocks, n_local_blocks, c_min, False)[0]


def retain_blocks_table(importance: torch.Tensor, block_size: int, n_real: int, budget: int,
                        n_sink_blocks: int = 1, n_local_blocks: int = 4, c_min: int = 1):
    """(mask [H, nb] bool, table [H, k] int32 ascending, lens [H] int32) of the
    retained set, from one launch and without a host sync."""
    return _retain(importance, block_size, n_real, budget, n_sink_blocks, n_local_blocks, c_min, True)


def h2o_retained_mask_torch(Q, K, block_size: int = 16, budget: int = 8, n_sink_blocks: int = 1,
                            n_local_blocks: int = 4, c_min: int = 1, chunk: int = 256) -> torch.Tensor:
    """Frozen H2O retained mask [H, nb] from the prompt (adakv/baselines_rt.py:130-143)."""
    imp = h2o_key_importance_torch(Q, K, chunk=chunk)
    return retain_blocks_torch(imp, block_size, K.shape[1], budget, n_sink_blocks, n_local_blocks, c_min)


def snapkv_retained_mask_torch(Q, K, block_size: int = 16, budget: int = 8, obs_window: int = 32,
                               pool_kernel: int = 7, n_sink_blocks: int = 1, n_local_blocks: int = 4,
                               c_min: int = 1) -> torch.Tensor:
    """Frozen SnapKV retained mask [H, nb] from the prompt (adakv/baselines_rt.py:146-159)."""
    imp = snapkv_key_importance_torch(Q, K, obs_window, pool_kernel)
    return retain_blocks_torch(imp, block_size, K.shape[1], budget, n_sink_blocks, n_local_blocks, c_min)


def _mask_table(mask: torch.Tensor, nb_now: int, n_sink_blocks: int, n_local_blocks: int):
    dev = _on_device(mask)
    if mask.dim() != 2 or mask.dtype not in (torch.bool, torch.uint8) or mask.stride(-1) != 1:
        raise ValueError("mask must be [H, nb] bool with a contiguous last axis")
    H, nbm = mask.shape
    table = torch.empty(H, nb_now, dtype=torch.int32, device=dev)
    lens = torch.empty(H, dtype=torch.int32, device=dev)
    sel = C.Selection(table.data_ptr(), nb_now, lens.data_ptr())
    C.check(C.load().adakv_mask_table(_ptr(mask), H, mask.stride(0), nbm, int(nb_now), int(n_sink_blocks),
                                      int(n_local_blocks), ctypes.byref(sel), _stream(dev)), "mask_table")
    k = int(lens.max().item())                   # the reference's host sync (baselines_rt.py:151)
    if not bool((lens == k).all()):
        raise AssertionError("mask_to_block_table expects an equal count per head")
    return table[:, :k].contiguous(), lens


def mask_to_block_table(mask: torch.Tensor):
    """(block_table [H, k] int32 ascending, sel_lens [H] int32) of a retained
    mask with an equal count per head (adakv/baselines_rt.py:139-155)."""
    return _mask_table(mask, mask.shape[1], 0, 0)


def frozen_decode_block_table(fmask: torch.Tensor, nb_now: int, n_sink_blocks: int, n_local_blocks: int):
    """Decode-step (block_table, sel_lens) of a frozen mask [H, nb_prefill]:
    the frozen blocks plus the sink and local blocks of ``nb_now`` blocks
    (adakv/baselines_rt.py:158-205)."""
    if nb_now < fmask.shape[1]:
        raise AssertionError("decode block count must not shrink below prefill")
    return _mask_table(fmask, nb_now, n_sink_blocks, n_local_blocks)


def frozen_table(table: torch.Tensor, lens: torch.Tensor, n_frozen_blocks: int, nb_now: int,
                 n_sink_blocks: int, n_local_blocks: int):
    """The decode-step table of a frozen set given as an ascending table
    [H, k] with lens [H] (as ``retain_blocks_table`` returns it): [H, width]
    int32 and lens, width = min(nb_now, k + sink + local); one launch, no
    host sync (the form the HuggingFace hook uses every step)."""
    dev = _on_device(table, lens)
    if table.dim() != 2 or table.dtype != torch.int32 or not table.is_contiguous():
        raise ValueError("table must be a contiguous [H, k] int32 tensor")
    if nb_now < n_frozen_blocks:
        raise AssertionError("decode block count must not shrink below prefill")
    H, k = table.shape
    width = max(1, min(int(nb_now), k + min(int(n_sink_blocks), nb_now) + min(int(n_local_blocks), nb_now)))
    out = torch.empty(H, width, dtype=torch.int32, device=dev)
    out_lens = torch.empty(H, dtype=torch.int32, device=dev)
    fsel = C.Selection(table.data_ptr(), k, lens.data_ptr())
    osel = C.Selection(out.data_ptr(), width, out_lens.data_ptr())
    C.check(C.load().adakv_frozen_table(ctypes.byref(fsel), H, int(n_frozen_blocks), int(nb_now),
                                        int(n_sink_blocks), int(n_local_blocks), ctypes.byref(osel), _stream(dev)),
            "frozen_table")
    return out, out_lens
