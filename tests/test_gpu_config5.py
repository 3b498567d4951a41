"""BASELINE config 5's attention shape through ``patch_model`` on the GPU
(adakv/patch.py:90-121): a random-init Llama with the 70B model's attention
-- 64 q / 8 KV heads, head_dim 128, hidden 8192 -- but a small MLP and
vocabulary and two layers, batch 4, a StaticCache of 65,536 tokens filled
directly with random bf16 K/V (no prefill, as ``bench.py --model-step``
does), avg_budget 8, three decode steps.

Every layer's decode step is checked where the hook launches it
(``hook_check.HookCheck``): the persistent summaries against a rebuild of
the live tokens (the first step builds them, the next two refresh them with
append_new), the selection of every sequence against the oracle's plan on
those summaries, and the output against fp64 attention over the GPU's
selection.  A full budget at the same head shape and a short context equals
SDPA.
"""
from __future__ import annotations

import pytest

from gpu_util import DEV, need_gpu, say, torch
from hook_check import HookCheck

pytestmark = pytest.mark.gpu

HQ, HKV, D, HIDDEN = 64, 8, 128, 8192


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    need_gpu()


def _model():
    from transformers import LlamaConfig, LlamaForCausalLM
    from adakv.patch import install_adakv
    cfg = LlamaConfig(vocab_size=256, hidden_size=HIDDEN, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D,
                      max_position_embeddings=131072, rope_theta=500000.0)
    torch.manual_seed(0)
    with torch.device(DEV):
        m = LlamaForCausalLM(cfg)
    m = m.to(dtype=torch.bfloat16).eval()
    install_adakv(m)
    return m, cfg


def _cfg(**kw):
    c = dict(block_size=16, avg_budget=8, k_min=2, k_max=64, n_sink_blocks=1, n_local_blocks=4,
             temperature=1.0, estimator="centroid", budget_policy="adaptive", c_min=1, nucleus_p=0.9,
             selection="adakv", centroid_dtype=None)
    c.update(kw)
    return c


def test_config5_shape_through_patch_model():
    from transformers import StaticCache
    from adakv.patch import enable_adakv
    B, S0, steps = 4, 65536, 3
    say(f"config 5 attention shape: {HQ}/{HKV} heads, D {D}, batch {B}, StaticCache {S0} tokens, "
        f"avg_budget 8, {steps} steps")
    model, cfg = _model()
    cache = StaticCache(config=cfg, max_cache_len=S0 + 16)
    gen = torch.Generator(device=DEV).manual_seed(5)
    kd = torch.zeros(B, HKV, 1, D, dtype=torch.bfloat16, device=DEV)
    for layer in cache.layers:
        layer.lazy_initialization(kd, kd)
        layer.keys[:, :, :S0].normal_(generator=gen)
        layer.values[:, :, :S0].normal_(generator=gen)
        if isinstance(layer.cumulative_length, torch.Tensor):
            layer.cumulative_length.fill_(S0)
        else:
            layer.cumulative_length = S0
    enable_adakv(**_cfg())
    with HookCheck() as hc:
        for i in range(steps):
            tok = torch.randint(0, cfg.vocab_size, (B, 1), device=DEV, generator=gen)
            pid = torch.full((B, 1), S0 + i, dtype=torch.long, device=DEV)
            with torch.no_grad():
                logits = model(input_ids=tok, position_ids=pid, past_key_values=cache, use_cache=True).logits
            assert torch.isfinite(logits).all()
    say(f"  {hc.calls} hook calls, {hc.sequences} sequences, {hc.heads - hc.excluded}/{hc.heads} heads "
        f"compared ({hc.excluded} near-ties), {hc.appends} incremental refreshes")
    assert hc.calls == 2 * steps and hc.sequences == 2 * steps * B
    assert hc.appends == 2 * (steps - 1)


def test_config5_shape_full_budget_equals_sdpa():
    """Every block selected: the patched model's decode logits equal SDPA's at
    the config-5 head shape (short context: SDPA holds the whole cache)."""
    from transformers import DynamicCache
    from adakv import attention as A
    from adakv.patch import disable_adakv, enable_adakv
    say("config 5 attention shape, full budget == SDPA (prompt 600, batch 2)")
    model, cfg = _model()
    gen = torch.Generator(device=DEV).manual_seed(6)
    ids = torch.randint(0, cfg.vocab_size, (2, 600), device=DEV, generator=gen)
    nxt = torch.randint(0, cfg.vocab_size, (2, 3), device=DEV, generator=gen)

    def run():
        cache = DynamicCache()
        out = []
        with torch.no_grad():
            model(input_ids=ids, past_key_values=cache, use_cache=True)
            for j in range(nxt.shape[1]):
                out.append(model(input_ids=nxt[:, j:j + 1], past_key_values=cache, use_cache=True).logits.float())
        return torch.cat(out, 1)

    enable_adakv(**_cfg(avg_budget=10 ** 6, k_min=10 ** 6, k_max=10 ** 6))
    A.reset_budget_trace()
    got = run()
    trace = A.get_budget_trace()
    A.stop_budget_trace()
    disable_adakv()
    ref = run()
    assert len(trace) == 2 * nxt.shape[1], "the HIP path did not run on every layer of every step"
    rel = ((got - ref).norm() / ref.norm()).item()
    say(f"  logits rel L2 {rel:.2e}")
    assert rel < 2e-2
