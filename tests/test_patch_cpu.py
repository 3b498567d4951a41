"""Host logic of the HuggingFace hook on the CPU: reading per-sequence runs
from HF's decode masks (adakv.patch._mask_runs), which decides between the
batched sparse path, the per-sequence path and SDPA, and the mask function
registered for the "adakv" attention implementation."""
from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")
pytest.importorskip("transformers")

from adakv import patch as P  # noqa: E402


def _mask(rows, kv_len, additive=False):
    """4-D decode mask [B, 1, 1, kv_len] from per-row attended index ranges."""
    m = torch.zeros(len(rows), 1, 1, kv_len, dtype=torch.bool)
    for b, spans in enumerate(rows):
        for lo, hi in spans:
            m[b, 0, 0, lo:hi] = True
    if additive:
        return torch.where(m, 0.0, float("-inf"))
    return m


def _runs(mask, B, kv_len):
    P._MASK_MEMO[0] = None            # every call here reads its own mask
    return P._mask_runs(mask, B, kv_len)


def test_prefix_runs_give_lengths_from_zero():
    starts, lens, lens_dev = _runs(_mask([[(0, 21)], [(0, 40)]], 64), 2, 64)
    assert starts == [0, 0] and lens == [21, 40]
    assert lens_dev.dtype == torch.int32 and lens_dev.tolist() == [21, 40]


def test_left_padding_gives_starts():
    starts, lens, _ = _runs(_mask([[(17, 300)], [(0, 300)], [(40, 300)]], 300), 3, 300)
    assert starts == [17, 0, 40] and lens == [283, 300, 260]


def test_additive_masks_are_read_like_boolean_ones():
    starts, lens, _ = _runs(_mask([[(3, 50)], [(0, 50)]], 64, additive=True), 2, 64)
    assert starts == [3, 0] and lens == [47, 50]


def test_a_row_with_a_hole_or_no_key_is_not_a_run():
    assert _runs(_mask([[(0, 20), (30, 64)], [(0, 64)]], 64), 2, 64) is None
    assert _runs(_mask([[], [(0, 64)]], 64), 2, 64) is None


def test_a_broadcast_batch_row_applies_to_every_sequence():
    starts, lens, lens_dev = _runs(_mask([[(0, 33)]], 48), 4, 48)
    assert starts == [0] * 4 and lens == [33] * 4 and lens_dev.numel() == 4


def test_shape_mismatches_are_not_runs():
    m = _mask([[(0, 10)], [(0, 10)]], 32)
    assert _runs(m, 2, 40) is None          # the keys have another length
    assert _runs(m, 3, 32) is None          # neither one row nor one per sequence


def test_the_layers_of_one_forward_read_a_mask_once():
    m = _mask([[(0, 12)]], 16)
    P._MASK_MEMO[0] = None
    first = P._mask_runs(m, 1, 16)
    assert P._MASK_MEMO[0] is m and P._mask_runs(m, 1, 16) is first


def test_the_adakv_implementation_has_an_sdpa_mask_function():
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, sdpa_mask
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    assert ALL_MASK_ATTENTION_FUNCTIONS["adakv"] is sdpa_mask
    assert "adakv" in ALL_ATTENTION_FUNCTIONS


def test_beam_reordering_permutes_each_layers_summaries():
    """Cache.reorder_cache (beam search) also permutes every layer state of the
    same batch: summaries, starts and lengths follow the beams, repeats
    included; a state of another batch size is left as it was."""
    from transformers import DynamicCache
    st = object.__new__(P._LayerState)
    st.centroid = torch.arange(3, dtype=torch.float32).view(3, 1, 1, 1).expand(3, 2, 4, 8).clone()
    st.starts, st.lens = [0, 1, 2], [10, 11, 12]
    other = object.__new__(P._LayerState)
    other.centroid = torch.zeros(2, 2, 4, 8)
    other.starts, other.lens = [0, 0], [5, 5]
    saved = dict(P._STATE)
    P._STATE.clear()
    P._STATE.update({1: st, 2: other})
    try:
        DynamicCache().reorder_cache(torch.tensor([2, 0, 0]))
    finally:
        P._STATE.clear()
        P._STATE.update(saved)
    assert st.centroid[:, 0, 0, 0].tolist() == [2.0, 0.0, 0.0]
    assert st.starts == [2, 0, 0] and st.lens == [12, 10, 10]
    assert other.lens == [5, 5] and not other.centroid.any()
