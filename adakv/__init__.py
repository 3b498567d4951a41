"""AdaKV on AMD Instinct MI355X (gfx950): the reference package's Python API.

Query-aware, per-head-adaptive block-sparse decode attention under the
reference's module names (``adakv.patch``, ``adakv.attention``,
``adakv.runtime``, ``adakv.kernels.block_sparse_decode``, ``adakv.baselines_rt``),
so that callers of the reference import this package unchanged.  The work runs
as hand-written HIP kernels in ``libadakv_amd.so`` (package ``adakv_amd``:
``csrc/`` sources, the ctypes binding of ``include/adakv_amd.h`` and the torch
wrappers in ``adakv_amd.ops``); there is no CPU fallback.
"""
__version__ = "0.2.0"
