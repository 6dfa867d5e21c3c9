"""The reference's Python boundary over the HIP library (needs a GPU):
``CAREKVLayer`` prefill / decode_step (layer.py:643-1163),
``patch_llama_model`` on a transformers LlamaForCausalLM
(llama_patch.py:112-359) and ``CAREKVAdapter`` (baselines/carekv_adapter.py).

Bars: the layer's prefill output matches the oracle's
``causal_attention_pure`` over the oracle's K_hat / V_hat followed by W_O
(fp32 on the CPU) within 2e-2 relative to the output scale (the projections
run in fp16 on the device); the cache the layer writes is byte-identical to
``write_prefill`` of the same K / V; the patched model's fp-mode logits
match the unpatched HF model's within 2e-2 of their scale.
"""
import math

import numpy as np
import pytest
import torch

from oracle import quant as Q
from oracle.attention import causal_attention_pure

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _cfg(L=1, Hq=8, Hkv=2, D=64, P=32, **kw):
    import care_kv
    base = dict(num_layers=L, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16, max_pages=P, base_bits=3,
                group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32, packed_base=True,
                scale_quant="int8", store_budget_mode="ratio", store_budget_ratio=0.03, read_budget_ratio=0.0)
    base.update(kw)
    return care_kv.CacheConfig(**base)


def _layer(cfg, model_dim, seed):
    import care_kv
    g = torch.Generator().manual_seed(seed)
    Hq, Hkv, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
    mk = lambda o, i: (torch.randn(o, i, generator=g) / math.sqrt(i)).half().cuda()  # noqa: E731
    return care_kv.CAREKVLayer(cfg, 0, mk(Hq * D, model_dim), mk(Hkv * D, model_dim), mk(Hkv * D, model_dim),
                               mk(model_dim, Hq * D))


@pytest.mark.parametrize("mode", ["fp", "base_quant"])
def test_layer_prefill_matches_oracle(monkeypatch, mode):
    import care_kv
    monkeypatch.setenv("CAREKV_PREFILL_MODE", mode)
    print(f"layer prefill mode={mode}", flush=True)
    cfg = _cfg()
    T, model_dim = 70, 256
    lay = _layer(cfg, model_dim, 3)
    hidden = (torch.randn(T, model_dim, generator=torch.Generator().manual_seed(4))).half().cuda()
    cache = care_kv.CAREKVCache(cfg, n_seq=1)
    out = lay.prefill(cache, hidden).float().cpu().numpy()
    # the oracle side: the same projections (same shapes as the layer's),
    # then layer.py:759-781 on the CPU
    Qt, Kt, Vt = lay._project(hidden.unsqueeze(0))
    Qd, Kd, Vd = Qt[0].cpu().numpy(), Kt[0].cpu().numpy(), Vt[0].cpu().numpy()
    Kraw, Vraw = Kt.contiguous(), Vt.contiguous()
    if mode == "base_quant":
        Kd = Q.dequantize(*Q.quantize(Kd, 3, 32), 32)
        Vd = Q.dequantize(*Q.quantize(Vd, 3, 32), 32)
    O, _ = causal_attention_pure(Qd, Kd, Vd)
    ref = O.transpose(1, 0, 2).reshape(T, -1).astype(np.float32) @ lay.W_O.float().cpu().numpy().T
    scale = float(np.abs(ref).max())
    assert np.abs(out - ref).max() <= 2e-2 * scale
    # the pages are those of write_prefill on the same post-RoPE K / V
    ref_cache = care_kv.CAREKVCache(cfg, n_seq=1)
    ref_cache.write_prefill(0, Kraw, Vraw, seqs=[0])
    for nm in ("kcodes", "vcodes", "kscale", "vscale", "kmaster", "vmaster", "valid", "k_slot", "v_slot"):
        assert torch.equal(getattr(cache, nm), getattr(ref_cache, nm)), nm


def test_layer_prefill_carekv_stored_matches_reference(monkeypatch):
    """CAREKVLayer.prefill in carekv_stored mode with correction_impl =
    vectorized (layer.py:538-557, 780-838; the golden's setting) on the
    reference prefill golden: identity projections pick q / k / v out of
    hidden = [q; k; v] and W_O returns the attention output (both exact in
    fp16), so the layer output is the corrected attention itself."""
    import care_kv
    from helpers import PAPER_ENV, PREFILL_CASES, load_golden, prefill_cfg_kwargs
    for k, v in PAPER_ENV.items():
        monkeypatch.setenv(k, v)
    monkeypatch.setenv("CAREKV_PREFILL_MODE", "carekv_stored")
    monkeypatch.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    print("layer prefill carekv_stored golden gqa8_d64", flush=True)
    g = load_golden("prefill_gqa8_d64.npz")
    spec = PREFILL_CASES["gqa8_d64"]
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0,
                              correction_impl="vectorized", **prefill_cfg_kwargs(g, spec))
    T, Hq, Hkv, D = int(g["T"]), spec["Hq"], spec["Hkv"], spec["D"]
    nq, nk = Hq * D, Hkv * D
    eye = torch.eye(nq + 2 * nk, dtype=torch.float16, device="cuda")
    lay = care_kv.CAREKVLayer(cfg, 0, eye[:nq].contiguous(), eye[nq:nq + nk].contiguous(),
                              eye[nq + nk:].contiguous(), eye[:nq, :nq].contiguous())
    Q, K, V = (torch.from_numpy(g[n]) for n in ("Q", "K", "V"))
    hidden = torch.cat([Q.reshape(T, -1), K.permute(1, 0, 2).reshape(T, -1), V.permute(1, 0, 2).reshape(T, -1)],
                       1).cuda()
    cache = care_kv.CAREKVCache(cfg, n_seq=1)
    out = lay.prefill(cache, hidden).float().cpu().numpy().reshape(T, Hq, D)
    ref = g["O"].astype(np.float32)
    err = np.abs(out - ref)
    assert np.all(err <= np.maximum(2e-3, np.spacing(np.abs(g["O"])).astype(np.float32))), err.max()


def test_layer_decode_steps_match_direct_calls(monkeypatch):
    """decode_step = append + decode_attention + W_O on the same cache."""
    import care_kv
    monkeypatch.setenv("CAREKV_PREFILL_MODE", "base_quant")
    print("layer decode steps", flush=True)
    cfg = _cfg()
    T, model_dim = 45, 256
    lay = _layer(cfg, model_dim, 5)
    g = torch.Generator().manual_seed(6)
    hidden = torch.randn(T + 3, model_dim, generator=g).half().cuda()
    cache = care_kv.CAREKVCache(cfg, n_seq=1)
    twin = care_kv.CAREKVCache(cfg, n_seq=1)
    lay.prefill(cache, hidden[:T])
    lay.prefill(twin, hidden[:T])
    for t in range(T, T + 3):
        out = lay.decode_step(cache, hidden[t:t + 1])
        Qt, Kt, Vt = lay._project(hidden[t:t + 1].unsqueeze(0))
        twin.append(0, Kt[:, :, 0], Vt[:, :, 0])
        o = care_kv.decode_attention(twin, 0, Qt[:, :, 0], correction=False)
        ref = lay._out(o.unsqueeze(2), o.dtype)[0]
        torch.testing.assert_close(out, ref, rtol=2e-3, atol=2e-3)
    assert cache.total_valid_tokens(0, 0) == T + 3


def _tiny_llama(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    c = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                    num_key_value_heads=2, vocab_size=1000, max_position_embeddings=1024)
    c._attn_implementation = "eager"
    return LlamaForCausalLM(c).half().cuda().eval()


def test_patched_llama_prefill_matches_hf(monkeypatch):
    import care_kv
    monkeypatch.setenv("CAREKV_PREFILL_MODE", "fp")
    print("patched llama prefill", flush=True)
    ids = torch.randint(0, 1000, (1, 48), generator=torch.Generator().manual_seed(1)).cuda()
    m = _tiny_llama()
    with torch.no_grad():
        ref = m(ids, use_cache=False).logits.float()
    cfg = _cfg(L=2, Hq=4, Hkv=2, D=64, P=16)
    care_kv.patch_llama_model(m, cfg)
    with torch.no_grad():
        got = m(ids, use_cache=False).logits.float()
    assert torch.isfinite(got).all()
    scale = float(ref.abs().max())
    assert float((got - ref).abs().max()) <= 2e-2 * scale


def test_patched_llama_generates_with_cache(monkeypatch):
    """greedy generate with use_cache=True: one prefill, then one decode
    step per new token through the CARE-KV cache (HF's cache length kept in
    step with zeros)."""
    import care_kv
    monkeypatch.setenv("CAREKV_PREFILL_MODE", "base_quant")
    print("patched llama generate", flush=True)
    ids = torch.randint(0, 1000, (1, 37), generator=torch.Generator().manual_seed(2)).cuda()
    m = _tiny_llama(1)
    cfg = _cfg(L=2, Hq=4, Hkv=2, D=64, P=16)
    care_kv.patch_llama_model(m, cfg)
    with torch.no_grad():
        out = m.generate(ids, max_new_tokens=5, do_sample=False, use_cache=True)
    assert out.shape == (1, 42)
    attn = [mod for mod in m.modules() if isinstance(mod, care_kv.CAREKVLlamaAttention)]
    cache = attn[0]._shared.cache
    for layer in range(2):
        assert cache.total_valid_tokens(layer, 0) == 41  # prompt + 4 decode appends
    care_kv.reset_all_caches(m)
    assert cache.total_valid_tokens(0, 0) == 0
    # HF's cache tracks the length only: one-wide placeholders, not a second KV cache
    from transformers import DynamicCache
    hf = DynamicCache()
    with torch.no_grad():
        m(ids, past_key_values=hf, use_cache=True)
    assert hf.get_seq_length() == 37
    assert all(lay.keys.shape[-1] == 1 for lay in getattr(hf, "layers", []))


def test_patched_llama_streaming_store(monkeypatch):
    """CAREKV_STREAMING_STORE=1: pages filled during generate get residual
    slots (the reference's fill store leaves them none)."""
    import care_kv
    monkeypatch.setenv("CAREKV_PREFILL_MODE", "base_quant")
    monkeypatch.setenv("CAREKV_STREAMING_STORE", "1")
    monkeypatch.setenv("CAREKV_STORE_POLICY", "residual_kind_aware")
    print("patched llama generate, streaming store", flush=True)
    ids = torch.randint(0, 1000, (2, 37), generator=torch.Generator().manual_seed(4)).cuda()
    m = _tiny_llama(2)
    cfg = _cfg(L=2, Hq=4, Hkv=2, D=64, P=16, store_budget_mode="absolute", store_abs_k=2, store_abs_v=4)
    care_kv.patch_llama_model(m, cfg)
    with torch.no_grad():
        out = m.generate(ids, max_new_tokens=30, do_sample=False, use_cache=True)
    assert out.shape == (2, 67)
    attn = [mod for mod in m.modules() if isinstance(mod, care_kv.CAREKVLlamaAttention)]
    cache = attn[0]._shared.cache
    assert cache.streaming_store
    # tokens 37..63 filled pages 2 and 3 during decode: both hold K slots now
    ks = cache.k_slot[0, 0, 0].cpu().numpy()
    assert (ks[2] >= 0).sum() == 2 and (ks[3] >= 0).sum() == 2
    care_kv.reset_all_caches(m)


def test_adapter_patches_a_given_model(monkeypatch):
    import care_kv
    import care_kv.layer
    print("adapter", flush=True)
    a = care_kv.CAREKVAdapter(sk=1, sv=1, rk=2, rv=2)
    for k, v in a.env().items():  # restored after the test
        monkeypatch.setenv(k, v)
    m = a.setup_model(_tiny_llama(2))
    ids = torch.randint(0, 1000, (1, 20), generator=torch.Generator().manual_seed(3)).cuda()
    import warnings
    with warnings.catch_warnings():
        warnings.simplefilter("error", RuntimeWarning)  # the default cached path is built: no fallback warning
        with torch.no_grad():
            logits = m(ids).logits
    assert torch.isfinite(logits.float()).all()
    st = a.collect_debug_stats()
    assert st["stored_k_slots"] > 0 and st["stored_v_slots"] > 0
    # the reference's gate for a CARE-KV row: slots were read (CLAUDE.md:141-142)
    assert st["k_reads"] > 0 and st["v_reads"] > 0


@pytest.mark.parametrize("name", ["gqa4_d128", "gqa4_d128_kivi"])
def test_layer_decode_step_matches_reference(monkeypatch, name):
    """CAREKVLayer.decode_step against the reference's own decode_step
    (layer.py:978-1163) on a decode golden: the prompt's pages, then 27
    decode steps whose appends fill the prompt's partial page and open two
    new pages (store on fill with K_orig = K_hat, zero master for the
    decode-opened page).  Identity projections pick q / k / v out of
    hidden = [q; k; v] and W_O returns the attention output, so the layer's
    last output is the reference's decode_step_out (read_budget_ratio = 0:
    the reference's decode attention is the base path, attention.py:1025)."""
    import care_kv
    from helpers import DECODE_CASES, PAPER_ENV, case_cfg_kwargs, load_golden
    for k, v in PAPER_ENV.items():
        monkeypatch.setenv(k, v)
    monkeypatch.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    print(f"layer decode_step golden {name}", flush=True)
    g = load_golden(f"decode_{name}.npz")
    spec = DECODE_CASES[name]
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0, compat=True,
                              **case_cfg_kwargs(g, spec))
    T, n_app = int(g["T"]), int(g["n_append"])
    Hq, Hkv, D = spec["Hq"], spec["Hkv"], spec["D"]
    nq, nk = Hq * D, Hkv * D
    eye = torch.eye(nq + 2 * nk, dtype=torch.float16, device="cuda")
    lay = care_kv.CAREKVLayer(cfg, 0, eye[:nq].contiguous(), eye[nq:nq + nk].contiguous(),
                              eye[nq + nk:].contiguous(), eye[:, :nq].contiguous())
    K, V, Qall = (torch.from_numpy(g[n]).cuda() for n in ("K", "V", "Qall"))
    cache = care_kv.CAREKVCache(cfg, n_seq=1)
    cache.write_prefill(0, K[:, :T], V[:, :T])
    out = None
    for i, t in enumerate(range(T, T + n_app)):
        hidden = torch.cat([Qall[i].reshape(-1), K[:, t].reshape(-1), V[:, t].reshape(-1)])[None]
        out = lay.decode_step(cache, hidden)
    got = out[0, :nq].reshape(Hq, D).float().cpu().numpy()
    ref = g["decode_step_out"].astype(np.float32)
    err = np.abs(got - ref)
    assert np.all(err <= np.maximum(2e-3, np.spacing(np.abs(g["decode_step_out"])).astype(np.float32))), err.max()
    # the cache after the appends equals the reference's, byte for byte
    from test_gpu_parity import compare_cache_to_golden
    compare_cache_to_golden(cache, g)


@pytest.mark.parametrize("name,Hq,D,k_mode,policy",
                         [("gqa4_d128", 8, 128, "exact", "joint"), ("gqa8_d64_linear", 16, 64, "linear", "separate")])
def test_layer_decode_step_corrected_matches_reference(monkeypatch, name, Hq, D, k_mode, policy):
    """compat=True: CAREKVLayer.decode_step with the reference's correction
    gate open (read_budget_ratio > 0, attention.py:1025) selects through the
    router's sketch-proxy score (apply_slot_corrections over
    ResidualRouter.route; CAREKV_KSCORE_LIVE=1 is set and ignored, as in the
    reference) and gives every one of the reference's decode steps within
    the decode bar: the prompt's partial page filled by the appends, a
    decode-opened page with its zero master, a page filled by decode."""
    import care_kv
    from helpers import PAPER_ENV, load_golden
    for k, v in PAPER_ENV.items():
        monkeypatch.setenv(k, v)
    monkeypatch.setenv("CAREKV_K_CORRECTION_MODE", k_mode)
    print(f"layer decode_step corrected golden {name}", flush=True)
    g = load_golden(f"decode_step_{name}.npz")
    T, n = int(g["T"]), int(g["n_append"])
    store = (dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4) if name == "gqa4_d128"
             else dict(store_budget_mode="ratio", store_budget_ratio=0.03))
    Hkv = 2
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                              max_pages=T // 16 + n // 16 + 4, base_bits=3, group_size=32, k_channel_group=32,
                              v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8",
                              read_budget_ratio=0.03, read_budget_mode="absolute", read_abs_k=int(g["read_k"]),
                              read_abs_v=int(g["read_v"]), route_policy=policy, compat=True, **store)
    nq, nk = Hq * D, Hkv * D
    eye = torch.eye(nq + 2 * nk, dtype=torch.float16, device="cuda")
    lay = care_kv.CAREKVLayer(cfg, 0, eye[:nq].contiguous(), eye[nq:nq + nk].contiguous(),
                              eye[nq + nk:].contiguous(), eye[:, :nq].contiguous())
    K, V, Qall = (torch.from_numpy(g[x]).cuda() for x in ("K", "V", "Qall"))
    cache = care_kv.CAREKVCache(cfg, n_seq=1)
    cache.write_prefill(0, K[:, :T], V[:, :T])
    for i, t in enumerate(range(T, T + n)):
        hidden = torch.cat([Qall[i].reshape(-1), K[:, t].reshape(-1), V[:, t].reshape(-1)])[None]
        got = lay.decode_step(cache, hidden)[0, :nq].reshape(Hq, D).float().cpu().numpy()
        ref = g["outs"][i]
        err = np.abs(got - ref.astype(np.float32))
        assert np.all(err <= np.maximum(2e-3, np.spacing(np.abs(ref)).astype(np.float32))), (i, err.max())
    from test_gpu_parity import compare_cache_to_golden
    compare_cache_to_golden(cache, g)
