"""AdaKV decode hot path for AMD Instinct MI355X (gfx950).

Query-aware, per-head-adaptive block-sparse decode attention: centroid block
scores, an entropy-driven per-head budget, top-k block selection and a ragged
split-K flash-decode, all as HIP kernels behind the C ABI in
``include/adakv_amd.h``.  The Python modules mirror the reference package's
API (``patch``, ``attention``, ``runtime``, ``kernels.block_sparse_decode``).
"""
__version__ = "0.1.0"
