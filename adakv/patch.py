"""Plug AdaKV into a HuggingFace model through the attention interface
(adakv/patch.py; transformers >= 5).

    from adakv.patch import patch_model
    patch_model(model, block_size=16, avg_budget=8)   # install + enable
    ... model.generate(...) ...
    disable_adakv()

Prefill (q_len > 1) and disabled calls go to HF's SDPA, as in the reference
(patch.py:96-100).  Single-token decode steps run the HIP pipeline with the
configured estimator ("centroid", or "minmax" for the Quest bound) and budget
policy.  Differences from the reference hook (patch.py:90-121):

* an SDPA-format mask function is registered for "adakv", so HF builds the
  masks SDPA would get (the reference registers none, and HF then passes no
  mask at all: padded batches and static caches were attended unmasked);
* each layer keeps its block summaries in HBM across steps and refreshes
  only the blocks that gained tokens (the reference rebuilds them from the
  whole cache every step, patch.py:110);
* batches of any size decode sparsely.  With no mask (a dynamic cache and an
  unpadded batch) every sequence holds the cache's length.  Otherwise each
  row of the decode mask must attend one contiguous run of keys, read from it
  once per forward (one host sync, shared by all layers): runs that all start
  at 0 (a static cache, whose unused tail is masked) decode as one batch with
  per-sequence lengths; runs that start later (left padding) decode one
  sequence at a time on its own view of the cache, so that its blocks count
  from its first real token, as for an unpadded sequence.  Any other mask goes
  to SDPA.

``selection="h2o"`` / ``"snapkv"`` selects the eviction baselines
(patch.py:57-87): on a single-sequence prefill that holds the whole prompt,
each layer freezes its retained block set from the prompt's attention (HIP
importance + retention; the prefill output itself is SDPA's), and each decode
step attends that set plus the current sink and local blocks through the
table-driven sparse decode.  As in the reference, batches of more than one
sequence go to SDPA, and a layer whose prefill was not seen attends every
block.
"""
from __future__ import annotations

import torch

from . import baselines_rt as _brt
from adakv_amd import ops
from .attention import instrumentation_active, record_selection

try:
    from transformers import AttentionInterface
except Exception:  # pragma: no cover - older transformers layouts
    from transformers.modeling_utils import AttentionInterface
from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

try:
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, sdpa_mask
except Exception:  # pragma: no cover - transformers without mask interfaces
    ALL_MASK_ATTENTION_FUNCTIONS = sdpa_mask = None

_ADAKV_CFG = dict(enabled=True, block_size=16, avg_budget=16, k_min=2, k_max=64,
                  n_sink_blocks=1, n_local_blocks=4, temperature=1.0,
                  estimator="centroid", budget_policy="adaptive",
                  c_min=1, nucleus_p=0.9,
                  selection="adakv", obs_window=32, pool_kernel=7, h2o_chunk=256,
                  centroid_dtype=None)
_SDPA = ALL_ATTENTION_FUNCTIONS["sdpa"]


class _LayerState:
    """Per-layer block summaries kept across decode steps: centroids
    [B, Hkv, capacity_blocks, D] or minmax bounds [B, Hkv, capacity_blocks, 2*D],
    built from tokens [starts[b], starts[b] + lens[b]) of sequence b."""

    def __init__(self, key, block_size, centroid_dtype, estimator, starts, lens, lens_dev):
        B, Hkv, S, D = key.shape
        nb = ops.n_blocks(S, block_size)
        cdt = _summary_dtype(key, centroid_dtype, estimator)
        self.sig = (B, Hkv, D, key.dtype, key.device, block_size, cdt, estimator)
        row = 2 * D if estimator == "minmax" else D
        self.centroid = torch.zeros(B, Hkv, nb + max(64, nb // 8), row, dtype=cdt, device=key.device)
        if not any(starts):
            ops.centroid_build(key, block_size, seq_lens=lens_dev, centroid=self.centroid, estimator=estimator)
        else:
            for b in range(B):
                ops.centroid_build(key[b:b + 1, :, starts[b]:starts[b] + lens[b]], block_size,
                                   centroid=self.centroid[b:b + 1], estimator=estimator)
        self.starts = list(starts)
        self.lens = list(lens)

    def grow(self, nb):
        if nb <= self.centroid.shape[2]:
            return
        c = self.centroid
        grown = torch.zeros(c.shape[0], c.shape[1], nb + max(64, nb // 8), c.shape[3], dtype=c.dtype,
                            device=c.device)
        grown[:, :, : c.shape[2]].copy_(c)
        self.centroid = grown


# Per-layer state keyed by id(module), like the reference's _FROZEN (patch.py:54).
_STATE: dict[int, _LayerState] = {}


def _reorder_states(beam_idx):
    """Beam search reorders the cache's rows between steps (Cache.reorder_cache,
    which generate() calls with the surviving beams, repeats allowed).  Each
    layer's summaries are kept per row, so they follow the same permutation:
    otherwise the next step would refresh only the newest block of every row
    and score the rest against another beam's summaries."""
    for st in _STATE.values():
        if st.centroid.shape[0] != beam_idx.numel():
            continue
        order = beam_idx.tolist()
        st.centroid = st.centroid.index_select(0, beam_idx.to(st.centroid.device))
        st.starts = [st.starts[i] for i in order]
        st.lens = [st.lens[i] for i in order]


def _wrap_reorder_cache():
    try:
        from transformers.cache_utils import Cache
    except Exception:  # pragma: no cover - transformers without the Cache class
        return
    if getattr(Cache.reorder_cache, "_adakv", False):
        return
    base = Cache.reorder_cache

    def reorder_cache(self, beam_idx):
        base(self, beam_idx)
        _reorder_states(beam_idx)

    reorder_cache._adakv = True
    Cache.reorder_cache = reorder_cache


_wrap_reorder_cache()

class _Frozen:
    """A layer's retained set, frozen at prefill: mask [Hq, nbp] bool and the
    same blocks as an ascending table [Hq, k] with lens [Hq]."""

    def __init__(self, mask, table, lens, nbp):
        self.mask, self.table, self.lens, self.nbp = mask, table, lens, nbp


# Eviction baselines' frozen sets keyed by id(module) (the reference's _FROZEN,
# patch.py:51-54); refreshed by every prefill, cleared by enable_adakv.
_FROZEN: dict[int, _Frozen] = {}
_ALL_BLOCKS: dict = {}


# The runs read from the last mask: (mask, result), so that the layers of one
# forward, which share one mask object, read it once.
_MASK_MEMO: list = [None, None]


def _mask_runs(mask, B, kv_len):
    """(host starts, host lengths, device int32 lengths) when every row of the
    decode mask (its last query row) attends one non-empty contiguous run of
    keys [start, start + length), else None."""
    if _MASK_MEMO[0] is mask:
        return _MASK_MEMO[1]
    res = None
    if mask.dim() == 4 and mask.shape[-1] == kv_len and mask.shape[0] in (1, B):
        m = mask[:, 0, -1, :]
        if m.dtype != torch.bool:
            m = m == 0                        # additive masks: 0 where attended
        lens = m.sum(-1)
        first = torch.argmax(m.to(torch.uint8), dim=-1)
        pos = torch.arange(kv_len, device=m.device)[None, :]
        ok = (m == ((pos >= first[:, None]) & (pos < (first + lens)[:, None]))).all()
        host = torch.cat([lens, first.to(lens.dtype), ok.view(1).to(lens.dtype)]).tolist()   # one host sync
        n = m.shape[0]
        lens_h, starts_h = [int(x) for x in host[:n]], [int(x) for x in host[n:2 * n]]
        if host[-1] and min(lens_h) >= 1:
            if n == 1 and B > 1:
                lens_h, starts_h = lens_h * B, starts_h * B
            res = (starts_h, lens_h, torch.tensor(lens_h, dtype=torch.int32, device=mask.device))
    _MASK_MEMO[0], _MASK_MEMO[1] = mask, res
    return res


def _summary_dtype(key, centroid_dtype, estimator):
    cdt = centroid_dtype or (torch.float32 if key.dtype == torch.float32 else key.dtype)
    if estimator == "minmax" and cdt not in (key.dtype, torch.float32):
        cdt = torch.float32          # minmax bounds stay exact: key dtype or fp32
    return cdt


def _signature(key, cfg):
    B, Hkv, S, D = key.shape
    cdt = _summary_dtype(key, cfg.get("centroid_dtype"), cfg["estimator"])
    return (B, Hkv, D, key.dtype, key.device, cfg["block_size"], cdt, cfg["estimator"])


def _budget(cfg):
    return ops.BudgetParams(avg_budget=cfg["avg_budget"], k_min=cfg["k_min"], k_max=cfg["k_max"],
                            n_sink_blocks=cfg["n_sink_blocks"],
                            n_local_blocks=cfg["n_local_blocks"], c_min=cfg["c_min"],
                            temperature=cfg["temperature"], budget_policy=cfg["budget_policy"],
                            nucleus_p=cfg.get("nucleus_p", 0.9))


def _prompt_len(key, attention_mask):
    """Tokens of the single sequence a forward sees: the mask's run when there
    is a mask (a static cache's unused tail is masked), else the key length.
    None when the mask row is not one run from position 0."""
    if attention_mask is None:
        return key.shape[2], None
    got = _mask_runs(attention_mask, 1, key.shape[2])
    if got is None or got[0][0] != 0:
        return None, None
    return got[1][0], got[2]


def _capture_frozen(module, query, key, attention_mask, cfg, sel):
    """Freeze this layer's retained blocks from the prompt (patch.py:57-73):
    per-q-head importance of the prompt's keys (H2O: every prompt query;
    SnapKV: the last obs_window queries, max-pooled), then the retained set.
    Only a forward that holds the whole prompt (its queries are every cached
    token) freezes a set; otherwise the layer keeps none and decodes over
    every block."""
    _FROZEN.pop(id(module), None)
    L, _ = _prompt_len(key, attention_mask)
    if L is None or L != query.shape[2]:
        return
    Q, K = query[0], key[0, :, :L]
    if sel == "h2o":
        imp = _brt.h2o_key_importance_torch(Q, K)
    else:
        imp = _brt.snapkv_key_importance_torch(Q, K, obs_window=int(cfg["obs_window"]),
                                               pool_kernel=int(cfg["pool_kernel"]))
    bs = int(cfg["block_size"])
    mask, table, lens = _brt.retain_blocks_table(imp, bs, L, int(cfg["avg_budget"]), cfg["n_sink_blocks"],
                                                 cfg["n_local_blocks"], cfg["c_min"])
    _FROZEN[id(module)] = _Frozen(mask, table, lens, ops.n_blocks(L, bs))


def _frozen_decode(module, query, key, value, attention_mask, scaling, cfg):
    """One decode step over the frozen set plus the current sink and local
    blocks (patch.py:76-87, 114-121); None when the mask is not a prefix run."""
    L, lens_dev = _prompt_len(key, attention_mask)
    if L is None:
        return None
    bs = int(cfg["block_size"])
    nb_now = ops.n_blocks(L, bs)
    Hq = query.shape[1]
    fr = _FROZEN.get(id(module))
    if fr is not None and fr.nbp <= nb_now:
        table, lens = _brt.frozen_table(fr.table, fr.lens, fr.nbp, nb_now, int(cfg["n_sink_blocks"]),
                                        int(cfg["n_local_blocks"]))
    else:                                        # prefill not seen: every block (patch.py:80-81)
        key_ = (query.device, Hq)
        empty = _ALL_BLOCKS.get(key_)
        if empty is None:
            empty = (torch.zeros(Hq, 1, dtype=torch.int32, device=query.device),
                     torch.zeros(Hq, dtype=torch.int32, device=query.device))
            _ALL_BLOCKS[key_] = empty
        table, lens = _brt.frozen_table(empty[0], empty[1], 0, nb_now, nb_now, 0)
    if instrumentation_active():
        record_selection(table, lens, nb_now)
    out = torch.empty(1, 1, Hq, query.shape[3], dtype=query.dtype, device=query.device)
    ops.sparse_decode(query[:, :, 0, :], key, value, table[None], lens[None], bs, sm_scale=scaling,
                      seq_lens=lens_dev, out=out[:, 0])
    return out


@torch.compiler.disable
def adakv_attention_forward(module, query, key, value, attention_mask, scaling, dropout=0.0,
                            **kwargs):
    """HF attention function (adakv/patch.py:90-121).

    query [B, Hq, q_len, D], key/value [B, Hkv, S, D] -> ([B, q_len, Hq, D], None).
    Excluded from torch.compile tracing (HF compiles the decode step of static
    caches): it launches through ctypes and keeps per-layer host state, so a
    compiled graph calls it as an opaque step.
    """
    cfg = _ADAKV_CFG
    B, Hq, q_len, D = query.shape
    sel = cfg.get("selection", "adakv")
    if sel not in ("adakv", "h2o", "snapkv"):
        raise ValueError(f"unknown selection: {sel!r}")
    if sel != "adakv":
        if cfg["enabled"] and B == 1 and q_len > 1:
            _capture_frozen(module, query, key, attention_mask, cfg, sel)   # the output stays dense
        elif cfg["enabled"] and B == 1:
            out = _frozen_decode(module, query, key, value, attention_mask, scaling, cfg)
            if out is not None:
                return out, None
        return _SDPA(module, query, key, value, attention_mask=attention_mask, scaling=scaling,
                     dropout=dropout, **kwargs)
    if (not cfg["enabled"]) or q_len != 1:
        if q_len != 1:
            _STATE.pop(id(module), None)        # a new prefill starts a new sequence
        return _SDPA(module, query, key, value, attention_mask=attention_mask, scaling=scaling,
                     dropout=dropout, **kwargs)
    if cfg["estimator"] not in ("centroid", "minmax"):
        raise ValueError(f"unknown estimator: {cfg['estimator']!r}")
    bs = int(cfg["block_size"])
    S = key.shape[2]
    if attention_mask is None:
        starts, lens, lens_dev = [0] * B, [S] * B, None
    else:
        got = _mask_runs(attention_mask, B, S)
        if got is None:                          # not one contiguous run per row
            return _SDPA(module, query, key, value, attention_mask=attention_mask, scaling=scaling,
                         dropout=dropout, **kwargs)
        starts, lens, lens_dev = got
    st = _STATE.get(id(module))
    append_new = None
    if st is not None and st.sig == _signature(key, cfg) and st.starts == starts:
        deltas = {n - p for n, p in zip(lens, st.lens)}
        if len(deltas) == 1 and min(deltas) >= 0:
            append_new = deltas.pop()
    if append_new is None:                       # new sequence(s): build from the cache
        st = _LayerState(key, bs, cfg.get("centroid_dtype"), cfg["estimator"], starts, lens, lens_dev)
        _STATE[id(module)] = st
        append_new = 0
    else:
        st.grow(ops.n_blocks(S, bs))
        st.lens = list(lens)
    out = torch.empty(B, 1, Hq, D, dtype=query.dtype, device=query.device)
    want = instrumentation_active()
    budget = _budget(cfg)
    if not any(starts):
        # a view of the tokens any row holds: a static cache larger than the
        # context is then scanned and selected over that context only
        n = max(max(lens), 1)
        if n < S:
            key, value = key[:, :, :n], value[:, :, :n]
        res = [ops.decode_fused(query[:, :, 0, :], key, value, st.centroid, bs, budget, seq_lens=lens_dev,
                                append_new=append_new, sm_scale=scaling, out=out[:, 0],
                                return_selection=want, estimator=cfg["estimator"])]
    else:
        # left padding: each sequence on its own view, tokens [start, start + length)
        res = [ops.decode_fused(query[b:b + 1, :, 0, :], key[b:b + 1, :, starts[b]:starts[b] + lens[b]],
                                value[b:b + 1, :, starts[b]:starts[b] + lens[b]], st.centroid[b:b + 1], bs,
                                budget, append_new=append_new, sm_scale=scaling, out=out[b:b + 1, 0],
                                return_selection=want, estimator=cfg["estimator"]) for b in range(B)]
    if want:
        record_selection(torch.cat([r[1] for r in res]), torch.cat([r[2] for r in res]),
                         ops.n_blocks(max(lens), bs))
    return out, None


AttentionInterface.register("adakv", adakv_attention_forward)
if ALL_MASK_ATTENTION_FUNCTIONS is not None:
    ALL_MASK_ATTENTION_FUNCTIONS.register("adakv", sdpa_mask)


def install_adakv(model):
    """Route the model's attention through "adakv" (adakv/patch.py:127-132)."""
    try:
        model.set_attn_implementation("adakv")
    except Exception:  # noqa: BLE001 - older models without the setter
        model.config._attn_implementation = "adakv"
    return model


def enable_adakv(**cfg):
    """Update the configuration and enable the sparse decode (adakv/patch.py:135-138)."""
    _ADAKV_CFG.update(cfg)
    _ADAKV_CFG["enabled"] = True
    _STATE.clear()
    _FROZEN.clear()                              # frozen sets of a previous configuration


def disable_adakv():
    _ADAKV_CFG["enabled"] = False


def patch_model(model, **cfg):
    """install_adakv + enable_adakv in one call (the README entry point,
    README.md:12-15, which the reference advertises but does not define)."""
    install_adakv(model)
    enable_adakv(**cfg)
    return model
