"""The C-ABI library on a CPU-only host: it loads, exports every symbol the
header declares, and rejects bad arguments on the host with the documented
status codes before touching a device."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from adakv_amd import _capi as C
from adakv_amd import ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "adakv_amd.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(C.lib_path()):
        pytest.skip("libadakv_amd.so not built (run python -m adakv_amd.build)")
    return C.load()


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(adakv_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    names = _declared()
    for n in ("adakv_centroid_build", "adakv_centroid_append", "adakv_plan", "adakv_sparse_decode",
              "adakv_decode_fused", "adakv_dense_decode", "adakv_workspace_bytes",
              "adakv_table_width"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    for n in _declared():
        assert hasattr(lib, n), n
        assert n in C.SIGNATURES, f"{n} has no ctypes signature"


def test_abi_version_and_status_strings(lib):
    assert lib.adakv_abi_version() == C.ABI_VERSION
    for s in range(9):
        assert lib.adakv_status_string(s) != b"unknown status"
    assert lib.adakv_status_string(99) == b"unknown status"


def _g(**kw):
    d = dict(B=1, Hq=32, Hkv=8, D=128, block_size=16, max_seq_len=131072, max_blocks=8192)
    d.update(kw)
    return C.Geometry(d["B"], d["Hq"], d["Hkv"], d["D"], d["block_size"], d["max_seq_len"],
                      d["max_blocks"])


def _b(**kw):
    return ops.BudgetParams(**kw).to_c()


def test_table_width_is_the_static_bound(lib):
    g = _g()
    assert lib.adakv_table_width(ctypes.byref(g), ctypes.byref(_b(avg_budget=8))) == 64
    assert lib.adakv_table_width(ctypes.byref(g), ctypes.byref(_b(k_max=2))) == 6   # sink+local+c_min
    assert lib.adakv_table_width(ctypes.byref(g), ctypes.byref(_b(k_max=100000))) == 8192
    small = _g(max_seq_len=40, max_blocks=3)
    assert lib.adakv_table_width(ctypes.byref(small), ctypes.byref(_b())) == 3


@pytest.mark.parametrize("bad,code", [
    (dict(Hq=30, Hkv=8), C.ADAKV_ERR_SHAPE),
    (dict(Hq=136, Hkv=8), C.ADAKV_ERR_UNSUPPORTED),      # group 17 > 16
    (dict(D=96), C.ADAKV_ERR_UNSUPPORTED),
    (dict(max_blocks=100), C.ADAKV_ERR_SHAPE),           # too few blocks for max_seq_len
    (dict(max_seq_len=65536 * 16, max_blocks=65536), C.ADAKV_ERR_UNSUPPORTED),
    (dict(B=0), C.ADAKV_ERR_SHAPE),
])
def test_geometry_validation(lib, bad, code):
    g = _g(**bad)
    q = C.Query(0x1000, C.ADAKV_BF16, 4096, 128)
    assert lib.adakv_dense_decode(ctypes.byref(g), ctypes.byref(q), None, None, ctypes.c_float(1.0),
                                  None, None, 0, None) == code
    assert lib.adakv_workspace_bytes(ctypes.byref(g), 64) == 0


def test_null_and_dtype_validation(lib):
    g = _g()
    kv = C.KV(0x1000, 0x2000, C.ADAKV_BF16, 0, 131072 * 128, 128)
    q = C.Query(0x1000, C.ADAKV_BF16, 4096, 128)
    out = C.Output(0x3000, C.ADAKV_BF16, 4096, 128)
    ws = ctypes.c_void_p(0x10000)
    f = lib.adakv_dense_decode
    assert f(ctypes.byref(g), None, ctypes.byref(kv), None, ctypes.c_float(1.0), ctypes.byref(out), ws,
             1 << 30, None) == C.ADAKV_ERR_NULL
    bad_q = C.Query(0x1000, 7, 4096, 128)
    assert f(ctypes.byref(g), ctypes.byref(bad_q), ctypes.byref(kv), None, ctypes.c_float(1.0),
             ctypes.byref(out), ws, 1 << 30, None) == C.ADAKV_ERR_DTYPE
    misaligned = C.KV(0x1002, 0x2000, C.ADAKV_BF16, 0, 131072 * 128, 128)
    assert f(ctypes.byref(g), ctypes.byref(q), ctypes.byref(misaligned), None, ctypes.c_float(1.0),
             ctypes.byref(out), ws, 1 << 30, None) == C.ADAKV_ERR_VALUE
    assert f(ctypes.byref(g), ctypes.byref(q), ctypes.byref(kv), None, ctypes.c_float(1.0),
             ctypes.byref(out), ws, 16, None) == C.ADAKV_ERR_WORKSPACE
    assert f(ctypes.byref(g), ctypes.byref(q), ctypes.byref(kv), None, ctypes.c_float(1.0),
             ctypes.byref(out), ctypes.c_void_p(0x10010), 1 << 30, None) == C.ADAKV_ERR_WORKSPACE
    assert f(ctypes.byref(g), ctypes.byref(q), ctypes.byref(kv), None, ctypes.c_float(float("nan")),
             ctypes.byref(out), ws, 1 << 30, None) == C.ADAKV_ERR_VALUE


def test_noalloc_refuses_a_step_larger_than_its_scratch(lib):
    """adakv_decode_fused_noalloc checks every argument and the step's scratch
    size on the host, before it looks up its static array or launches: here a
    geometry of 64 sequences of 131072 tokens (whose fp32 scores alone exceed
    ADAKV_NOALLOC_SCRATCH_BYTES) and argument errors come back on a CPU host."""
    big = _g(B=64)
    assert lib.adakv_workspace_bytes(ctypes.byref(big), 64) > C.NOALLOC_SCRATCH_BYTES
    q = C.Query(0x1000, C.ADAKV_BF16, 4096, 128)
    kv = C.KV(0x1000, 0x2000, C.ADAKV_BF16, 8 * 131072 * 128, 131072 * 128, 128)
    c = C.Centroid(0x4000, C.ADAKV_BF16, C.SUMMARY_CENTROID)
    out = C.Output(0x3000, C.ADAKV_BF16, 4096, 128)
    f = lib.adakv_decode_fused_noalloc
    bud = _b(avg_budget=8)
    assert f(ctypes.byref(big), ctypes.byref(q), ctypes.byref(kv), ctypes.byref(c), None, ctypes.byref(bud),
             None, 1, ctypes.c_float(0.088), ctypes.byref(out), None) == C.ADAKV_ERR_SCRATCH
    assert b"ADAKV_NOALLOC_SCRATCH_BYTES" in lib.adakv_status_string(C.ADAKV_ERR_SCRATCH)
    g = _g()
    assert f(ctypes.byref(g), None, ctypes.byref(kv), ctypes.byref(c), None, ctypes.byref(bud),
             None, 1, ctypes.c_float(0.088), ctypes.byref(out), None) == C.ADAKV_ERR_NULL
    assert f(ctypes.byref(g), ctypes.byref(q), ctypes.byref(kv), ctypes.byref(c), None, ctypes.byref(bud),
             None, -1, ctypes.c_float(0.088), ctypes.byref(out), None) == C.ADAKV_ERR_VALUE
    narrow = C.Selection(0x5000, 8, 0x6000)
    assert f(ctypes.byref(g), ctypes.byref(q), ctypes.byref(kv), ctypes.byref(c), None, ctypes.byref(bud),
             ctypes.byref(narrow), 1, ctypes.c_float(0.088), ctypes.byref(out), None) == C.ADAKV_ERR_SHAPE


def test_scan_launch_validates_on_the_host(lib):
    """adakv_decode_fused_scan (the step's first launch alone) rejects bad
    arguments before any launch, as adakv_decode_fused does."""
    g = _g()
    q = C.Query(0x1000, C.ADAKV_BF16, 4096, 128)
    kv = C.KV(0x1000, 0x2000, C.ADAKV_BF16, 8 * 131072 * 128, 131072 * 128, 128)
    c = C.Centroid(0x4000, C.ADAKV_BF16, C.SUMMARY_CENTROID)
    bud = _b(avg_budget=8)
    ws = ctypes.c_void_p(0x10000)
    f = lib.adakv_decode_fused_scan
    assert f(ctypes.byref(g), None, ctypes.byref(kv), ctypes.byref(c), None, ctypes.byref(bud), 1, ws, 1 << 30,
             None) == C.ADAKV_ERR_NULL
    assert f(ctypes.byref(g), ctypes.byref(q), ctypes.byref(kv), ctypes.byref(c), None, ctypes.byref(bud), -1,
             ws, 1 << 30, None) == C.ADAKV_ERR_VALUE
    assert f(ctypes.byref(g), ctypes.byref(q), ctypes.byref(kv), ctypes.byref(c), None, ctypes.byref(bud), 1,
             ws, 16, None) == C.ADAKV_ERR_WORKSPACE
    # an append needs the centroid type to pair with K's: fp16 K, bf16 centroids
    f16kv = C.KV(0x1000, 0x2000, C.ADAKV_F16, 8 * 131072 * 128, 131072 * 128, 128)
    assert f(ctypes.byref(g), ctypes.byref(q), ctypes.byref(f16kv), ctypes.byref(c), None, ctypes.byref(bud), 1,
             ws, 1 << 30, None) == C.ADAKV_ERR_DTYPE


def test_plan_validation(lib):
    g = _g()
    q = C.Query(0x1000, C.ADAKV_BF16, 4096, 128)
    c = C.Centroid(0x4000, C.ADAKV_BF16)
    ws = ctypes.c_void_p(0x10000)
    sel = C.Selection(0x5000, 64, 0x6000)
    narrow = C.Selection(0x5000, 8, 0x6000)
    bad_policy = C.Budget(8.0, 2, 64, 1, 4, 1, 1.0, 5)
    nan_nucleus = C.Budget(8.0, 2, 64, 1, 4, 1, 1.0, C.POLICY_NUCLEUS, float("nan"))
    neg = C.Budget(8.0, 2, -1, 1, 4, 1, 1.0, 1)
    ok = _b(avg_budget=8)
    f = lib.adakv_plan
    args = lambda b, s: (ctypes.byref(g), ctypes.byref(q), ctypes.byref(c), None, ctypes.byref(b),
                         ctypes.byref(s), ws, 1 << 30, None)
    assert f(*args(bad_policy, sel)) == C.ADAKV_ERR_VALUE
    assert f(*args(nan_nucleus, sel)) == C.ADAKV_ERR_VALUE
    assert f(*args(neg, sel)) == C.ADAKV_ERR_VALUE
    assert f(*args(ok, narrow)) == C.ADAKV_ERR_SHAPE
    nullsel = C.Selection(0, 64, 0x6000)
    assert f(*args(ok, nullsel)) == C.ADAKV_ERR_NULL


def test_centroid_dtype_pairs(lib):
    g = _g()
    kv = C.KV(0x1000, 0, C.ADAKV_F16, 0, 131072 * 128, 128)
    c = C.Centroid(0x4000, C.ADAKV_BF16)
    assert lib.adakv_centroid_build(ctypes.byref(g), ctypes.byref(kv), None, ctypes.byref(c),
                                    None) == C.ADAKV_ERR_DTYPE
    c2 = C.Centroid(0x4000, C.ADAKV_F16)
    assert lib.adakv_centroid_append(ctypes.byref(g), ctypes.byref(kv), None, 0, ctypes.byref(c2),
                                     None) == C.ADAKV_ERR_VALUE          # n_new must be >= 1


def test_minmax_summary_validation(lib):
    """Summary kinds: an unknown kind is a bad value, minmax rows need head_dim
    <= 128 and an exact element type (the key type or fp32)."""
    kv32 = C.KV(0x1000, 0, C.ADAKV_F32, 0, 131072 * 128, 128)
    kv16 = C.KV(0x1000, 0, C.ADAKV_BF16, 0, 131072 * 128, 128)
    g = _g()
    build = lambda geo, kv, c: lib.adakv_centroid_build(ctypes.byref(geo), ctypes.byref(kv), None,
                                                        ctypes.byref(c), None)
    assert build(g, kv16, C.Centroid(0x4000, C.ADAKV_BF16, 7)) == C.ADAKV_ERR_VALUE
    assert build(g, kv32, C.Centroid(0x4000, C.ADAKV_BF16, C.SUMMARY_MINMAX)) == C.ADAKV_ERR_DTYPE
    assert build(g, kv16, C.Centroid(0x4000, C.ADAKV_F16, C.SUMMARY_MINMAX)) == C.ADAKV_ERR_DTYPE
    g256 = _g(D=256, Hq=8, Hkv=8)
    assert build(g256, kv16, C.Centroid(0x4000, C.ADAKV_BF16, C.SUMMARY_MINMAX)) == \
        C.ADAKV_ERR_UNSUPPORTED
    q = C.Query(0x1000, C.ADAKV_BF16, 4096, 128)
    assert lib.adakv_block_scores(ctypes.byref(g256), ctypes.byref(q),
                                  ctypes.byref(C.Centroid(0x4000, C.ADAKV_F32, C.SUMMARY_MINMAX)),
                                  None, ctypes.c_void_p(0x8000), 8192, None) == C.ADAKV_ERR_UNSUPPORTED


def test_summary_kind_from_the_row_length():
    """ops infers the estimator from the summary's last dimension."""
    import torch
    assert ops.summary_kind(torch.zeros(1, 2, 4, 64), 64) == "centroid"
    assert ops.summary_kind(torch.zeros(1, 2, 4, 128), 64) == "minmax"
    assert ops.summary_kind(torch.zeros(1, 2, 4, 128), 64, "minmax") == "minmax"
    with pytest.raises(ValueError):
        ops.summary_kind(torch.zeros(1, 2, 4, 64), 64, "minmax")
    with pytest.raises(ValueError):
        ops.summary_kind(torch.zeros(1, 2, 4, 96), 64)
    with pytest.raises(ValueError):
        ops.summary_kind(torch.zeros(1, 2, 4, 64), 64, "bogus")


def test_workspace_bytes_grows_with_the_problem(lib):
    small, big = _g(max_seq_len=4096, max_blocks=256), _g()
    assert 0 < lib.adakv_workspace_bytes(ctypes.byref(small), 64) < \
        lib.adakv_workspace_bytes(ctypes.byref(big), 64)
    assert lib.adakv_workspace_bytes(ctypes.byref(big), 0) == 0


def test_python_errors_mirror_the_reference(lib):
    """Unknown estimator / policy -> ValueError; CPU tensors -> RuntimeError
    (the reference raises RuntimeError without its GPU kernel)."""
    import torch

    from adakv.attention import AdaKVCache, plan_selection
    from adakv.kernels.block_sparse_decode import block_sparse_decode
    with pytest.raises(ValueError):
        AdaKVCache(16, estimator="bogus")
    cache = AdaKVCache(16)
    with pytest.raises(RuntimeError):
        cache.append_prefill(torch.zeros(2, 64, 32), torch.zeros(2, 64, 32))
    with pytest.raises(ValueError):
        plan_selection(torch.zeros(4, 32), cache, 8, estimator="nope")
    with pytest.raises(ValueError):
        plan_selection(torch.zeros(4, 32), cache, 8, budget_policy="nope")
    with pytest.raises(ValueError):
        plan_selection(torch.zeros(4, 32), cache, 8, estimator="minmax")
    with pytest.raises(RuntimeError):
        AdaKVCache(16, estimator="minmax").append_prefill(torch.zeros(2, 64, 32), torch.zeros(2, 64, 32))
    assert ops.BudgetParams(budget_policy="adaptive_nucleus", nucleus_p=0.8).to_c().policy == \
        C.POLICY_NUCLEUS
    with pytest.raises(ValueError):
        ops.BudgetParams(budget_policy="nucleus").to_c()
    with pytest.raises(RuntimeError):
        block_sparse_decode(torch.zeros(4, 32), torch.zeros(2, 64, 32), torch.zeros(2, 64, 32),
                            torch.zeros(4, 2, dtype=torch.int32), torch.ones(4, dtype=torch.int32), 16)


def test_eviction_entry_points_validate_on_the_host(lib):
    """The eviction-baseline entry points reject bad arguments before any
    launch (no device needed)."""
    P = C.Prompt

    def prompt(**kw):
        d = dict(q=0x1000, k=0x2000, dtype=C.ADAKV_BF16, Hq=32, Hkv=8, D=128, L=8192,
                 qsh=8192 * 128, qss=128, ksh=8192 * 128, kss=128)
        d.update(kw)
        return P(d["q"], d["k"], d["dtype"], d["Hq"], d["Hkv"], d["D"], d["L"], d["qsh"], d["qss"], d["ksh"],
                 d["kss"])

    ws = lib.adakv_importance_workspace_bytes
    assert ws(ctypes.byref(prompt()), 0) == 32 * 8192 * 4
    # 32 queries, G 4: 8 grouped waves x 2 tile groups = 16 waves, split 32 ways over 8192 keys (256 each)
    assert ws(ctypes.byref(prompt()), 8192 - 32) == 32 * 32 * 4 + 32 * 32 * 32 * 8
    assert ws(ctypes.byref(prompt()), 8192) == 0                      # no query left
    assert ws(ctypes.byref(prompt(D=96)), 0) == 0

    def imp(p, first=0, pitch=8192, nbytes=32 * 8192 * 4, scale=0.088):
        return lib.adakv_key_importance(ctypes.byref(p), first, ctypes.c_float(scale), ctypes.c_void_p(0x9000),
                                        pitch, ctypes.c_void_p(0xA000), nbytes, None)
    assert imp(prompt(Hkv=5)) == C.ADAKV_ERR_SHAPE
    assert imp(prompt(dtype=9)) == C.ADAKV_ERR_DTYPE
    assert imp(prompt(D=256)) == C.ADAKV_ERR_UNSUPPORTED
    assert imp(prompt(q=0x1004)) == C.ADAKV_ERR_VALUE                 # misaligned rows
    assert imp(prompt(qss=100)) == C.ADAKV_ERR_VALUE
    assert imp(prompt(), pitch=8000) == C.ADAKV_ERR_SHAPE
    assert imp(prompt(), first=-1) == C.ADAKV_ERR_VALUE
    assert imp(prompt(), scale=float("nan")) == C.ADAKV_ERR_VALUE
    assert imp(prompt(), nbytes=1024) == C.ADAKV_ERR_WORKSPACE
    assert imp(prompt(k=0)) == C.ADAKV_ERR_NULL

    pool = lib.adakv_importance_pool
    assert pool(ctypes.c_void_p(0x1000), ctypes.c_void_p(0x100000), 4, 100, 100, 4, None) == C.ADAKV_ERR_VALUE
    assert pool(ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1100), 4, 100, 100, 7, None) == C.ADAKV_ERR_VALUE
    assert pool(ctypes.c_void_p(0x1000), ctypes.c_void_p(0x100000), 4, 100, 50, 7, None) == C.ADAKV_ERR_SHAPE

    def retain(n_real=8192, bs=16, mask_pitch=512, budget=8, sel=None):
        return lib.adakv_retain_blocks(ctypes.c_void_p(0x1000), 32, 1 << 20, n_real, bs, budget, 1, 4, 1,
                                       ctypes.c_void_p(0x2000), mask_pitch, sel, None)
    assert retain(n_real=16 * 16385, mask_pitch=16385) == C.ADAKV_ERR_UNSUPPORTED
    assert retain(mask_pitch=511) == C.ADAKV_ERR_SHAPE
    assert retain(budget=-1) == C.ADAKV_ERR_VALUE
    narrow = C.Selection(0x3000, 7, 0x4000)                            # k = 8 does not fit
    assert retain(sel=ctypes.byref(narrow)) == C.ADAKV_ERR_SHAPE

    frozen = C.Selection(0x3000, 8, 0x4000)
    out = C.Selection(0x5000, 12, 0x6000)
    ft = lib.adakv_frozen_table
    assert ft(ctypes.byref(frozen), 32, 512, 511, 1, 4, ctypes.byref(out), None) == C.ADAKV_ERR_SHAPE
    assert ft(ctypes.byref(frozen), 32, 512, 600, 1, 4, ctypes.byref(C.Selection(0x5000, 12, 0x6000)),
              None) == C.ADAKV_ERR_SHAPE                               # needs 8 + 1 + 4
    assert ft(ctypes.byref(frozen), 32, 512, 70000, 1, 4, ctypes.byref(C.Selection(0x5000, 13, 0x6000)),
              None) == C.ADAKV_ERR_UNSUPPORTED
    mt = lib.adakv_mask_table
    assert mt(ctypes.c_void_p(0x1000), 32, 512, 512, 512, 0, 0, ctypes.byref(C.Selection(0x5000, 511, 0x6000)),
              None) == C.ADAKV_ERR_SHAPE
    assert mt(None, 32, 512, 512, 512, 0, 0, ctypes.byref(out), None) == C.ADAKV_ERR_NULL
