"""A patched random-init LLaMA with the CARE-KV correction on, against an
oracle-driven forward of the same weights (needs a GPU).

The patched model (patch_llama_model, carekv_stored prefill with the
vectorized query-aware correction, the default decode path: correction on
under a read budget, re-encoding appends and the streaming fill store) and a
copy whose attention modules run the CPU oracle instead (the same torch
projections and RoPE, then oracle write_pages_for_kv_head + prefill_stored
for the prompt, decode_append(streaming, rescale) + decode_attention for
each new token) see the same token stream: a prompt whose last page is
partial, then decode tokens that fill it and open a new page.

Bars: every layer's attention output (before W_O) of the patched model
within max-abs 2e-3 (or one fp16 ulp) of the oracle run on the same layer
inputs (the patched model's, replayed call by call), with no warning
raised; the logits of the free-running oracle model within 5e-2 of the
logits' scale of the patched model's at every position (their layer inputs
drift apart by fp16 roundings, which can move a selection across a tie).
"""
import warnings

import numpy as np
import pytest
import torch
from torch import nn

from helpers import PAPER_ENV
from oracle.attention import decode_attention as oracle_decode
from oracle.attention import prefill_stored
from oracle.cache import OCache, OCfg
from oracle.store import decode_append, write_pages_for_kv_head

pytestmark = pytest.mark.gpu
F16, F32 = np.float16, np.float32

CARE = dict(num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64, page_size=16, max_pages=8, base_bits=3,
            group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32, store_budget_mode="absolute",
            store_abs_k=2, store_abs_v=4, read_budget_mode="absolute", read_abs_k=2, read_abs_v=2,
            route_policy="joint")


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _model(seed=3):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    c = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                    num_key_value_heads=2, vocab_size=1000, max_position_embeddings=1024, initializer_range=0.05)
    c._attn_implementation = "eager"
    return LlamaForCausalLM(c).half().cuda().eval()


class OracleAttention(nn.Module):
    """The oracle's attention in place of a LlamaAttention: the patched
    layer's own projections and RoPE (torch, same weights), the CPU oracle
    for the cache and the attention, W_O in torch."""

    def __init__(self, W_Q, W_K, W_V, W_O, layer_id, log):
        super().__init__()
        import care_kv
        self.layer = care_kv.CAREKVLayer(care_kv.CacheConfig(**CARE), layer_id, W_Q, W_K, W_V, W_O)
        self.layer_id, self.log, self.oc = layer_id, log, None

    def forward(self, hidden_states, attention_mask=None, position_ids=None, past_key_values=None, use_cache=False,
                cache_position=None, position_embeddings=None, **kw):
        from care_kv.layer import _rope
        B, T, _ = hidden_states.shape
        Q, K, V = self.layer._project(hidden_states)
        cos, sin = position_embeddings
        Q, K = _rope(Q, K, cos.to(Q.dtype), sin.to(Q.dtype))
        Qn, Kn, Vn = (x[0].half().cpu().numpy() for x in (Q, K, V))
        kw_corr = dict(k_mode="exact", kind="both", k_corr_scale=0.1, score_normalize=True, kscore_live=True)
        if T > 1:
            self.oc = OCache(OCfg(**dict(CARE, num_layers=1)))
            hats = [write_pages_for_kv_head(self.oc, 0, h, Kn[h], Vn[h]) for h in range(2)]
            kh, vh = np.stack([a for a, _ in hats]), np.stack([b for _, b in hats])
            O = prefill_stored(self.oc, 0, Qn, kh, vh, **kw_corr)                 # (T, Hq, D)
        else:
            decode_append(self.oc, 0, Kn[:, 0], Vn[:, 0], streaming=True, rescale=True)
            O = oracle_decode(self.oc, 0, Qn[:, 0], **kw_corr)[None]              # (1, Hq, D)
        self.log.append((self.layer_id, T, O))
        Ot = torch.from_numpy(O).cuda().transpose(0, 1)[None]                     # (1, Hq, T, D)
        out = self.layer._out(Ot, hidden_states.dtype).to(hidden_states.dtype)
        if use_cache and past_key_values is not None:
            z = hidden_states.new_zeros((B, 2, T, 1))
            past_key_values.update(z, z, self.layer_id)
        return out, None


def test_patched_llama_with_correction_matches_oracle_forward(monkeypatch):
    import care_kv
    from transformers import DynamicCache
    for k, v in PAPER_ENV.items():
        monkeypatch.setenv(k, v)
    monkeypatch.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    monkeypatch.setenv("CAREKV_PREFILL_MODE", "carekv_stored")
    print("patched llama with correction vs oracle forward", flush=True)
    T, n_dec = 44, 6  # the prompt's third page holds 12 rows; decode fills it at token 47 and opens page 4
    ids = torch.randint(0, 1000, (1, T + n_dec), generator=torch.Generator().manual_seed(9)).cuda()
    patched, oracle_m = _model(), _model()
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0,
                              correction_impl="vectorized", **CARE)
    care_kv.patch_llama_model(patched, cfg)
    got_log, inputs = [], []
    for mod in patched.modules():
        if isinstance(mod, care_kv.CAREKVLlamaAttention):
            lay = mod.care_layer
            orig_out = lay._out

            def rec(O, dtype, _lid=mod.layer_id, _f=orig_out):
                got_log.append((_lid, O.shape[2], O[0].transpose(0, 1).float().cpu().numpy()))
                return _f(O, dtype)
            lay._out = rec

            def pre(m_, args, kwargs, _lid=mod.layer_id):
                hs = args[0] if args else kwargs["hidden_states"]
                inputs.append((_lid, hs.detach().clone(), tuple(x.detach().clone()
                                                              for x in kwargs["position_embeddings"])))
            mod.register_forward_pre_hook(pre, with_kwargs=True)
    ref_log = []
    for i, layer in enumerate(oracle_m.model.layers):
        a_ = layer.self_attn
        layer.self_attn = OracleAttention(a_.q_proj.weight.data, a_.k_proj.weight.data, a_.v_proj.weight.data,
                                          a_.o_proj.weight.data, i, ref_log)
    logits_got, logits_ref = [], []
    with torch.no_grad(), warnings.catch_warnings():
        warnings.simplefilter("error")
        for m, out in ((patched, logits_got), (oracle_m, logits_ref)):
            pkv = DynamicCache()
            out.append(m(ids[:, :T], past_key_values=pkv, use_cache=True).logits[0].float())
            for t in range(T, T + n_dec):
                out.append(m(ids[:, t:t + 1], past_key_values=pkv, use_cache=True).logits[0].float())
    assert len(got_log) == len(ref_log) == len(inputs) == 2 * (1 + n_dec)
    # teacher forced: the oracle on the patched model's own layer inputs
    replay_log = []
    lays = {mod.layer_id: mod.care_layer for mod in patched.modules()
            if isinstance(mod, care_kv.CAREKVLlamaAttention)}
    replay = [OracleAttention(lays[i].W_Q, lays[i].W_K, lays[i].W_V, lays[i].W_O, i, replay_log) for i in range(2)]
    with torch.no_grad():
        for lid, hs, pe in inputs:
            replay[lid](hs, position_embeddings=pe)
    for (lg, tg, og), (lr, tr, orf) in zip(got_log, replay_log):
        assert (lg, tg) == (lr, tr)
        err = np.abs(og - orf.astype(F32))
        bar = np.maximum(2e-3, np.spacing(np.abs(orf)).astype(F32))
        assert np.all(err <= bar), (lg, tg, float(err.max()))
    worst = 0.0
    for a, b in zip(logits_got, logits_ref):
        worst = max(worst, float((a - b).abs().max()) / float(b.abs().max()))
    print(f"free-running logits: worst max-abs difference {worst:.2e} of the logits' scale", flush=True)
    assert worst <= 5e-2
    # the decode steps corrected (the default mode): slots were selected
    cache = next(mod for mod in patched.modules() if isinstance(mod, care_kv.CAREKVLlamaAttention))._shared.cache
    assert cache.streaming_store and cache.rescale_open
    assert int((cache.k_slot[0, 0, 0, 2] >= 0).sum()) == 2  # the refilled third page got slots from its true rows
