"""Block-sparse flash-decode on MI355X (adakv/kernels/block_sparse_decode.py:103-135).

``block_sparse_decode`` keeps the reference's signature and shapes; the work is
the ragged split-K HIP kernel of ``libadakv_amd.so``.  Batched inputs (a
leading batch axis on every argument) are accepted as an extension.

Inputs (decode, one query token per sequence):
    q            [n_q_heads, head_dim]                fp32 / fp16 / bf16
    k_cache      [n_kv_heads, seq_len, head_dim]      head_dim contiguous
    v_cache      [n_kv_heads, seq_len, head_dim]
    block_table  [n_q_heads, max_sel]   int32         selected block ids per head
    sel_lens     [n_q_heads]            int32         valid entries per row
Output:
    out          [n_q_heads, head_dim]  (q dtype)
"""
from __future__ import annotations

from adakv_amd import _capi, ops

#: True when the HIP library is built and a ROCm device is visible.
HAS_HIP = False
try:  # pragma: no cover - depends on the host
    import torch as _torch
    HAS_HIP = _capi.available() and _torch.cuda.is_available()
except Exception:  # noqa: BLE001
    HAS_HIP = False

#: The reference exports ``HAS_TRITON`` (patch.py:34, runtime.py:23); callers
#: that test it keep working: it reports whether the GPU kernel path is usable.
HAS_TRITON = HAS_HIP


def block_sparse_decode(q, k_cache, v_cache, block_table, sel_lens, block_size, sm_scale=None,
                        seq_lens=None):
    """Attention of each q-head over exactly its listed KV blocks.

    Raises RuntimeError for CPU tensors or a missing library (the reference
    raises RuntimeError when Triton is absent, block_sparse_decode.py:108-112).
    """
    if k_cache.dim() == 3:
        out = ops.sparse_decode(q.unsqueeze(0), k_cache.unsqueeze(0), v_cache.unsqueeze(0),
                                block_table.unsqueeze(0).contiguous(),
                                sel_lens.unsqueeze(0).contiguous(), block_size, sm_scale)
        return out[0]
    return ops.sparse_decode(q, k_cache, v_cache, block_table.contiguous(), sel_lens.contiguous(),
                             block_size, sm_scale, seq_lens=seq_lens)
