"""Model-agnostic decode runtime (adakv/runtime.py).

``update_cache_decode`` appends one token's KV in place and refreshes the
trailing block centroid on the GPU; ``adakv_decode_step`` plans and runs the
sparse decode.  Prefill stays dense and is not part of this package (the
reference's ``dense_prefill``, runtime.py:26-40, is a plain torch einsum).
There is no CPU backend: the reference's pure-torch fallback
(runtime.py:63-82) is replaced by the NumPy oracle used in tests.
"""
from __future__ import annotations

from .attention import AdaKVCache, adakv_decode_attention

__all__ = ["update_cache_decode", "adakv_decode_step"]


def update_cache_decode(cache: AdaKVCache, k_t, v_t):
    """Append one decoded token's KV (k_t, v_t: [Hkv, 1, D]) and refresh the
    block centroid it lands in (adakv/runtime.py:43-60)."""
    return cache.append_decode(k_t, v_t)


def adakv_decode_step(q, cache: AdaKVCache, avg_budget, k_min: int = 2, k_max: int = 64,
                      n_sink_blocks: int = 1, n_local_blocks: int = 4, temperature: float = 1.0,
                      backend: str = "auto"):
    """One AdaKV decode step.  q: [1, Hq, 1, D] -> [1, Hq, 1, D] (adakv/runtime.py:85-112).

    ``backend``: "auto" / "hip" run the HIP kernels ("triton" is accepted as the
    reference's name for the GPU kernel); "torch" (the reference's CPU
    fallback) is not provided.
    """
    assert q.shape[0] == 1, "runtime currently supports batch size 1 (use adakv_amd.ops for B>1)"
    if backend == "torch":
        raise NotImplementedError("no CPU decode backend: AdaKV runs as HIP kernels only")
    if backend not in ("auto", "hip", "triton"):
        raise ValueError(f"unknown backend: {backend!r}")
    out = adakv_decode_attention(q[0, :, 0, :], cache, avg_budget, k_min, k_max, n_sink_blocks,
                                 n_local_blocks, temperature)
    return out.unsqueeze(0).unsqueeze(2)
