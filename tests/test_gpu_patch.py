"""The HuggingFace drop-in (adakv/patch.py:90-138) on the GPU: a small
random-init Llama routed through ``patch_model``.

* With a budget that selects every block, the sparse decode is attention over
  the whole cache, so the patched model's decode logits must equal the
  unpatched (SDPA) model's -- the reference's full-budget check
  (tests/test_reference.py:71-79) at the model level, covering RoPE, GQA,
  the softmax scale and the output layout.  fp32 (three-kernel path) and bf16
  (fused path), centroid and minmax estimators, adaptive and nucleus budgets.
* Dynamic and static caches, batch 1 and 2: the HIP path runs (the budget
  trace records every layer of every step), with the static cache's lengths
  taken from its mask.
* A left-padded batch (each mask row one contiguous run that starts late):
  every sequence decodes on its own view of the cache, blocks counted from its
  first real token; with every block selected it equals SDPA over the mask.
* A mask row that is not one contiguous run goes to SDPA.
* A normal budget: the realised mean budget is the requested one.
* The eviction baselines (selection "h2o" / "snapkv"): a full budget equals
  SDPA, a normal budget keeps the frozen count, batches go to SDPA.
"""
from __future__ import annotations

import pytest

from gpu_util import DEV, need_gpu, say, torch
from hook_check import HookCheck

pytestmark = pytest.mark.gpu

VOCAB, PROMPT, STEPS = 256, 300, 4


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    need_gpu()


def _model(dtype):
    from transformers import LlamaConfig, LlamaForCausalLM
    from adakv.patch import install_adakv
    cfg = LlamaConfig(vocab_size=VOCAB, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                      max_position_embeddings=4096)
    torch.manual_seed(0)
    m = LlamaForCausalLM(cfg).to(device=DEV, dtype=dtype).eval()
    install_adakv(m)
    return m


FULL = dict(avg_budget=10 ** 6, k_min=10 ** 6, k_max=10 ** 6)


def _cfg(**kw):
    c = dict(block_size=16, avg_budget=8, k_min=2, k_max=64, n_sink_blocks=1, n_local_blocks=4,
             temperature=1.0, estimator="centroid", budget_policy="adaptive", c_min=1, nucleus_p=0.9,
             selection="adakv", centroid_dtype=None)
    c.update(kw)
    return c


def _decode_logits(model, ids, cache_kind, attention_mask=None):
    """Prefill `ids`, then STEPS single-token steps of fixed tokens; the logits of each step."""
    from transformers import StaticCache
    B = ids.shape[0]
    cache = None
    if cache_kind == "static":
        cache = StaticCache(config=model.config, max_cache_len=PROMPT + STEPS + 37)
    out = []
    with torch.no_grad():
        r = model(ids, attention_mask=attention_mask, past_key_values=cache, use_cache=True)
        cache = r.past_key_values
        am = attention_mask
        for t in range(STEPS):
            tok = torch.full((B, 1), (7 * t + 3) % VOCAB, dtype=torch.long, device=DEV)
            if am is not None:
                am = torch.cat([am, torch.ones(B, 1, dtype=am.dtype, device=DEV)], dim=1)
            r = model(tok, attention_mask=am, past_key_values=cache, use_cache=True)
            out.append(r.logits[:, -1].float())
    return torch.stack(out)


def _run(model, ids, cache_kind, cfg, attention_mask=None):
    """(patched logits, unpatched logits, layer-steps recorded by the HIP path)."""
    from adakv import attention as A
    from adakv.patch import disable_adakv, enable_adakv
    disable_adakv()
    ref = _decode_logits(model, ids, cache_kind, attention_mask)
    enable_adakv(**cfg)
    A.reset_budget_trace()
    got = _decode_logits(model, ids, cache_kind, attention_mask)
    trace = A.get_budget_trace()
    A.stop_budget_trace()
    disable_adakv()
    torch.cuda.synchronize()
    return got, ref, trace


def _ids(B):
    g = torch.Generator().manual_seed(1)
    return torch.randint(0, VOCAB, (B, PROMPT), generator=g).to(DEV)


@pytest.mark.parametrize("cache_kind", ["dynamic", "static"])
@pytest.mark.parametrize("B", [1, 2])
def test_full_budget_equals_sdpa_fp32(cache_kind, B):
    say(f"patch fp32 full budget, {cache_kind} cache, B={B}")
    model = _model(torch.float32)
    got, ref, trace = _run(model, _ids(B), cache_kind, _cfg(**FULL))
    assert len(trace) == STEPS * 2, "the HIP path did not run on every layer of every step"
    err = (got - ref).abs().max().item()
    say(f"  max |logit diff| {err:.2e}")
    assert err <= 2e-3 * max(ref.abs().max().item(), 1.0)


@pytest.mark.parametrize("est,policy", [("centroid", "adaptive"), ("minmax", "fixed"),
                                        ("centroid", "adaptive_nucleus")])
@pytest.mark.parametrize("cache_kind", ["dynamic", "static"])
def test_full_budget_equals_sdpa_bf16(cache_kind, est, policy):
    say(f"patch bf16 full budget, {cache_kind} cache, {est}/{policy}")
    model = _model(torch.bfloat16)
    got, ref, trace = _run(model, _ids(2), cache_kind, _cfg(estimator=est, budget_policy=policy, **FULL))
    assert len(trace) == STEPS * 2
    rel = ((got - ref).norm() / ref.norm()).item()
    say(f"  logits rel L2 {rel:.2e}")
    assert rel < 2e-2


def _left_padded(B=3):
    am = torch.ones(B, PROMPT, dtype=torch.long, device=DEV)
    am[0, :17] = 0
    am[2, :40] = 0
    return am


@pytest.mark.parametrize("cache_kind", ["dynamic", "static"])
def test_left_padded_batch_full_budget_equals_sdpa(cache_kind):
    say(f"patch left-padded batch of 3, fp32 full budget, {cache_kind} cache")
    model = _model(torch.float32)
    got, ref, trace = _run(model, _ids(3), cache_kind, _cfg(**FULL), attention_mask=_left_padded())
    assert len(trace) == STEPS * 2, "the HIP path did not run on every layer of every step"
    err = (got - ref).abs().max().item()
    say(f"  max |logit diff| {err:.2e}")
    assert err <= 2e-3 * max(ref.abs().max().item(), 1.0)


def test_left_padded_batch_bf16_normal_budget():
    say("patch left-padded batch of 3, bf16, avg_budget 8")
    model = _model(torch.bfloat16)
    got, ref, trace = _run(model, _ids(3), "dynamic", _cfg(avg_budget=8), attention_mask=_left_padded())
    assert len(trace) == STEPS * 2
    assert all(abs(t - 8.0) <= 0.5 for t in trace), trace
    assert torch.isfinite(got).all()


def test_non_contiguous_mask_goes_to_sdpa():
    """A mask row with a hole is not one run: the hook hands the step to SDPA."""
    say("patch mask with a hole -> SDPA")
    model = _model(torch.bfloat16)
    am = torch.ones(2, PROMPT, dtype=torch.long, device=DEV)
    am[1, 100:110] = 0
    got, ref, trace = _run(model, _ids(2), "dynamic", _cfg(), attention_mask=am)
    assert len(trace) == 0, "a mask with a hole must not take the sparse path"
    assert torch.equal(got, ref)


@pytest.mark.parametrize("cache_kind", ["dynamic", "static"])
def test_normal_budget_realises_the_mean(cache_kind):
    say(f"patch bf16 avg_budget 8, {cache_kind} cache")
    model = _model(torch.bfloat16)
    got, ref, trace = _run(model, _ids(2), cache_kind, _cfg(avg_budget=8))
    assert len(trace) == STEPS * 2
    assert all(abs(t - 8.0) <= 0.5 for t in trace), trace
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("cache_kind", ["dynamic", "static"])
def test_normal_budget_hook_steps_match_the_oracle(cache_kind):
    """avg_budget 8 over STEPS steps: at every layer and step the hook's
    persistent summaries equal a rebuild of the live tokens (the first step
    builds them, later steps refresh them through append_new, a static cache
    through its views of the live tokens), the selection equals the oracle's
    plan on them, and the output equals fp64 attention over it."""
    from adakv.patch import disable_adakv, enable_adakv
    say(f"patch bf16 avg_budget 8, {cache_kind} cache: every hook step against the oracle")
    model = _model(torch.bfloat16)
    enable_adakv(**_cfg(avg_budget=8))
    with HookCheck() as hc:
        _decode_logits(model, _ids(2), cache_kind)
    disable_adakv()
    say(f"  {hc.calls} hook calls, {hc.heads - hc.excluded}/{hc.heads} heads compared")
    assert hc.calls == STEPS * 2 and hc.sequences == STEPS * 2 * 2
    assert hc.appends == (STEPS - 1) * 2


def test_left_padded_normal_budget_hook_steps_match_the_oracle():
    """A left-padded batch at avg_budget 8: each sequence decodes on its own
    view (blocks counted from its first real token), and its summaries,
    selection and output hold at every layer and step."""
    from adakv.patch import disable_adakv, enable_adakv
    say("patch left-padded batch of 3, bf16 avg_budget 8: every hook step against the oracle")
    model = _model(torch.bfloat16)
    enable_adakv(**_cfg(avg_budget=8))
    with HookCheck() as hc:
        _decode_logits(model, _ids(3), "dynamic", attention_mask=_left_padded())
    disable_adakv()
    assert hc.calls == STEPS * 2 * 3 and hc.appends == (STEPS - 1) * 2 * 3


def test_beam_search_keeps_each_rows_summaries():
    """generate(num_beams=2) at avg_budget 8: beam search reorders the cache's
    rows between steps (Cache.reorder_cache); the layers' summaries follow the
    same permutation, so every step's summaries equal a rebuild of each row's
    tokens and its selection matches the oracle.  48 new tokens: the beams'
    own tokens reach blocks that the step's append no longer recomputes, so
    summaries left unpermuted would show."""
    from adakv.patch import disable_adakv, enable_adakv
    say("patch generate(num_beams=2, 48 tokens), bf16 avg_budget 8: summaries follow the beams")
    model = _model(torch.bfloat16)
    ids = _ids(1)
    new = 48
    enable_adakv(**_cfg(avg_budget=8))
    with HookCheck() as hc:
        with torch.no_grad():
            model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=new, min_new_tokens=new,
                           num_beams=2, do_sample=False, pad_token_id=0)
    disable_adakv()
    say(f"  {hc.calls} hook calls, {hc.appends} incremental refreshes")
    assert hc.calls == (new - 1) * 2 and hc.sequences == (new - 1) * 2 * 2
    assert hc.appends == (new - 2) * 2


def test_generate_with_static_cache_matches_sdpa_greedy():
    """model.generate with an HF StaticCache (the usage INTEGRATION.md shows):
    with a budget that selects every block the greedy continuation equals the
    unpatched model's, and every decode step ran on the HIP path."""
    from transformers import StaticCache
    from adakv import attention as A
    from adakv.patch import disable_adakv, enable_adakv
    say("patch generate() with StaticCache, fp32, full budget")
    model = _model(torch.float32)
    ids = _ids(2)
    new = 6

    def gen():
        cache = StaticCache(config=model.config, max_cache_len=PROMPT + new + 40)
        with torch.no_grad():
            return model.generate(ids, attention_mask=torch.ones_like(ids), past_key_values=cache,
                                  max_new_tokens=new, do_sample=False, pad_token_id=0)

    disable_adakv()
    ref = gen()
    enable_adakv(**_cfg(**FULL))
    A.reset_budget_trace()
    got = gen()
    trace = A.get_budget_trace()
    A.stop_budget_trace()
    disable_adakv()
    assert len(trace) == (new - 1) * 2, f"{len(trace)} layer-steps on the HIP path"
    assert torch.equal(got, ref)


@pytest.mark.parametrize("sel", ["h2o", "snapkv"])
@pytest.mark.parametrize("cache_kind", ["dynamic", "static"])
def test_eviction_full_budget_equals_sdpa(sel, cache_kind):
    """selection="h2o"/"snapkv" (adakv/patch.py:57-87): a budget that retains
    every block freezes the whole prompt, so decoding over the frozen set plus
    the new tail equals SDPA; every decode step ran on the HIP path."""
    say(f"patch {sel} fp32 full budget, {cache_kind} cache")
    model = _model(torch.float32)
    got, ref, trace = _run(model, _ids(1), cache_kind, _cfg(selection=sel, **FULL))
    assert len(trace) == STEPS * 2, "the frozen decode did not run on every layer of every step"
    err = (got - ref).abs().max().item()
    say(f"  max |logit diff| {err:.2e}")
    assert err <= 2e-3 * max(ref.abs().max().item(), 1.0)


@pytest.mark.parametrize("sel", ["h2o", "snapkv"])
def test_eviction_normal_budget_keeps_the_frozen_count(sel):
    """avg_budget 8: every head keeps 8 frozen blocks of the 19-block prompt;
    the decode tokens stay inside the last block, so each step attends 8."""
    say(f"patch {sel} bf16 avg_budget 8")
    model = _model(torch.bfloat16)
    got, ref, trace = _run(model, _ids(1), "dynamic", _cfg(selection=sel, avg_budget=8))
    assert trace == [8.0] * (STEPS * 2), trace
    assert torch.isfinite(got).all()
    rel = ((got - ref).norm() / ref.norm()).item()
    say(f"  logits rel L2 vs dense {rel:.2e}")


def test_eviction_batches_go_to_sdpa():
    """As in the reference (patch.py:96-100), the eviction baselines decode
    single sequences only; a batch of two is SDPA's."""
    say("patch h2o, batch of 2 -> SDPA")
    model = _model(torch.bfloat16)
    got, ref, trace = _run(model, _ids(2), "dynamic", _cfg(selection="h2o"))
    assert len(trace) == 0
    assert torch.equal(got, ref)
