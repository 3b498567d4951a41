"""Native AdaKV decode library for AMD Instinct MI355X (gfx950).

``csrc/`` holds the HIP kernels and the C ABI of ``include/adakv_amd.h``
(centroid build and append, block scores, budget, selection, sparse and dense
flash-decode, the fused decode step, the eviction baselines), built in-tree
into ``_lib/libadakv_amd.so`` by ``adakv_amd.build``.  ``_capi`` binds it with
ctypes and ``ops`` wraps it for torch tensors.  The reference's Python API
(``adakv.patch``, ``adakv.attention``, ...) lives in the package ``adakv``.
"""
__version__ = "0.2.0"
