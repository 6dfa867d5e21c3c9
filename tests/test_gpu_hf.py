"""HF integration of the patched model (llama_patch.py:112-359) on the GPU:
the CARE-KV HF cache object and padded batch prompts.

Bars: greedy generation through the default ``CAREKVHFCache`` gives the
same tokens and the same per-step logits, bit for bit, as the same model fed
a caller's DynamicCache (the one-wide placeholder path); a left-padded batch
of prompts of different lengths generates, row by row, the tokens each
prompt generates alone, with per-step logits within 1e-3 of their scale
(1e-2 with the correction on: the batched fp16 projections of HF's layers
round differently from a batch of one, and a selection can then cross a
tie), and no pad row reaches a page.  The patched model itself is held to the
oracle in tests/test_gpu_e2e.py; these tests hold its batching and cache
plumbing to that same single-sequence path.
"""
import pytest
import torch

from helpers import PAPER_ENV

pytestmark = pytest.mark.gpu

CARE = dict(num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64, page_size=16, max_pages=8, base_bits=3,
            group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8",
            store_budget_mode="absolute", store_abs_k=2, store_abs_v=4, read_budget_mode="absolute", read_abs_k=2,
            read_abs_v=2, route_policy="joint", read_budget_ratio=0.0, correction_impl="vectorized")


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _patched(monkeypatch, correction: bool, seed=5):
    import care_kv
    from transformers import LlamaConfig, LlamaForCausalLM
    if correction:
        for k, v in PAPER_ENV.items():
            monkeypatch.setenv(k, v)
        monkeypatch.setenv("CAREKV_K_CORRECTION_MODE", "exact")
        monkeypatch.setenv("CAREKV_PREFILL_MODE", "carekv_stored")
        cfg = care_kv.CacheConfig(**CARE)
    else:
        monkeypatch.setenv("CAREKV_PREFILL_MODE", "base_quant")
        cfg = care_kv.CacheConfig(**dict(CARE, read_budget_mode="ratio"))
    torch.manual_seed(seed)
    c = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                    num_key_value_heads=2, vocab_size=1000, max_position_embeddings=1024, initializer_range=0.05)
    m = LlamaForCausalLM(c).half().cuda().eval()
    care_kv.patch_llama_model(m, cfg)
    return m


def _gen(m, ids, n, **kw):
    with torch.no_grad():
        return m.generate(ids, max_new_tokens=n, do_sample=False, use_cache=True, return_dict_in_generate=True,
                          output_logits=True, pad_token_id=0, **kw)


@pytest.mark.parametrize("correction", [False, True], ids=["base", "corrected"])
def test_carekv_hf_cache_matches_placeholder_path(monkeypatch, correction):
    import care_kv
    from transformers import DynamicCache
    print(f"CAREKVHFCache vs DynamicCache placeholders, correction={correction}", flush=True)
    m = _patched(monkeypatch, correction)
    ids = torch.randint(1, 1000, (2, 45), generator=torch.Generator().manual_seed(6)).cuda()
    a = _gen(m, ids, 8)
    assert isinstance(a.past_key_values, care_kv.CAREKVHFCache)
    shared = next(mod for mod in m.modules() if isinstance(mod, care_kv.CAREKVLlamaAttention))._shared
    assert a.past_key_values.care_cache is shared.cache
    assert [a.past_key_values.get_seq_length(i) for i in range(2)] == [52, 52]
    for layer in range(2):
        assert shared.cache.total_valid_tokens(layer, 1, seq=1) == 52
    b = _gen(m, ids, 8, past_key_values=DynamicCache())
    assert type(b.past_key_values) is DynamicCache
    assert torch.equal(a.sequences, b.sequences)
    for la, lb in zip(a.logits, b.logits):
        assert torch.equal(la, lb)


@pytest.mark.parametrize("correction", [False, True], ids=["base", "corrected"])
def test_left_padded_batch_matches_single_prompts(monkeypatch, correction):
    import care_kv
    print(f"left-padded batch vs single prompts, correction={correction}", flush=True)
    m = _patched(monkeypatch, correction)
    lens, n_new = [40, 27, 9], 10
    T = max(lens)
    g = torch.Generator().manual_seed(7)
    prompts = [torch.randint(1, 1000, (n,), generator=g) for n in lens]
    ids = torch.zeros((len(lens), T), dtype=torch.long)
    mask = torch.zeros((len(lens), T), dtype=torch.long)
    for b, p in enumerate(prompts):
        ids[b, T - len(p):] = p
        mask[b, T - len(p):] = 1
    out = _gen(m, ids.cuda(), n_new, attention_mask=mask.cuda())
    shared = next(mod for mod in m.modules() if isinstance(mod, care_kv.CAREKVLlamaAttention))._shared
    for b, n in enumerate(lens):  # the pad rows never reached a page
        for layer in range(2):
            for h in range(2):
                assert shared.cache.total_valid_tokens(layer, h, seq=b) == n + n_new - 1
    worst = 0.0
    for b, p in enumerate(prompts):
        one = _gen(m, p[None].cuda(), n_new)
        assert torch.equal(out.sequences[b, T:], one.sequences[0, len(p):]), b
        for lb, l1 in zip(out.logits, one.logits):
            d = float((lb[b].float() - l1[0].float()).abs().max()) / float(l1[0].float().abs().max())
            worst = max(worst, d)
    print(f"worst per-step logit difference {worst:.2e} of the logits' scale", flush=True)
    assert worst <= (1e-2 if correction else 1e-3)
