"""CPU tests: the C-ABI library loads and exports every declared symbol, and the
host-side knob resolution matches the reference's budget arithmetic."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _ensure_built():
    from care_kv import _lib
    if not os.path.exists(_lib.lib_path()):
        from care_kv.build import build
        build()
    return _lib


def test_library_exports_header_symbols():
    _lib = _ensure_built()
    lib = _lib.load()
    hdr = open(os.path.join(ROOT, "include", "carekv.h")).read()
    declared = set(re.findall(r"\b(carekv_[a-z0-9_]+)\s*\(", hdr))
    assert declared, "no declarations parsed"
    for name in sorted(declared):
        assert hasattr(lib, name), name
    assert set(_lib.EXPORTS) <= declared


def _struct_fields(hdr, name):
    body = hdr[hdr.index(f"typedef struct {name}"):hdr.index(f"}} {name};")]
    body = re.sub(r"/\*.*?\*/", " ", body, flags=re.S)
    body = body[body.index("{") + 1:]
    names = []
    for stmt in body.split(";"):
        stmt = stmt.strip()
        if not stmt:
            continue
        decl = re.sub(r"^(const\s+)?(unsigned\s+)?(long\s+)*\w+\s*", "", stmt)  # drop the type
        names += [re.sub(r"[\s*]", "", d) for d in decl.split(",")]
    return names


def test_c_structs_match_header_layout():
    """ctypes mirrors of the C structs have the header's field order."""
    _lib = _ensure_built()
    hdr = open(os.path.join(ROOT, "include", "carekv.h")).read()
    for cname, py in (("carekv_arena", _lib.Arena), ("carekv_store_params", _lib.StoreParams),
                      ("carekv_decode_params", _lib.DecodeParams), ("carekv_prefill_params", _lib.PrefillParams),
                      ("carekv_prefill_eval_params", _lib.PrefillEvalParams),
                      ("carekv_prefill_grid", _lib.PrefillGrid)):
        assert [f[0] for f in py._fields_] == _struct_fields(hdr, cname), cname


def test_cpu_tensor_is_rejected():
    _lib = _ensure_built()
    import torch
    with pytest.raises(_lib.CarekvError):
        _lib.ptr(torch.zeros(3))


def test_unsupported_config_rejected():
    import care_kv
    from care_kv.cache import check_kernel_config
    with pytest.raises(NotImplementedError):
        check_kernel_config(care_kv.CacheConfig(page_size=8, group_size=32, base_bits=3))
    with pytest.raises(NotImplementedError):  # rotation bases are not built
        check_kernel_config(care_kv.CacheConfig(base_quantizer="rotatekv_style", group_size=32))
    with pytest.raises(NotImplementedError):  # pre-RoPE KVQuant is not built
        check_kernel_config(care_kv.CacheConfig(base_quantizer="kvquant_style", k_store_mode="pre_rope",
                                                group_size=32))
    check_kernel_config(care_kv.CacheConfig(group_size=32, base_bits=3, head_dim=128))
    check_kernel_config(care_kv.CacheConfig(base_quantizer="kivi_style", group_size=32, base_bits=2))


def test_config_validation_matches_reference():
    import care_kv
    with pytest.raises(ValueError):
        care_kv.CacheConfig(scale_quant="int4")
    with pytest.raises(ValueError):
        care_kv.CacheConfig(route_policy="greedy")
    c = care_kv.CacheConfig(num_heads=8, packed_storage=True)
    assert c.num_kv_heads == 8 and c.packed_base and c.layer_sensitivity == [1.0] * 32


def test_store_knobs(monkeypatch):
    """Ratio 3% at D=128 resolves to 1 K + 1 V slot per page
    (residual_store.py:403-408); absolute mode passes the counts through."""
    import care_kv
    monkeypatch.delenv("CAREKV_STORE_POLICY", raising=False)
    monkeypatch.delenv("CAREKV_PREFILL_RESIDUAL_KIND", raising=False)
    c = care_kv.CacheConfig(num_layers=1, head_dim=128, group_size=32, store_budget_mode="ratio",
                            store_budget_ratio=0.03)
    s = care_kv.resolve_store_knobs(c, 0)
    assert (s.k_budget, s.v_budget, s.joint, s.store_none) == (1, 1, False, False)
    c = care_kv.CacheConfig(num_layers=1, group_size=32, store_budget_mode="absolute", store_abs_k=2,
                            store_abs_v=4, store_budget_ratio=0.0)
    s = care_kv.resolve_store_knobs(c, 0)
    assert (s.k_budget, s.v_budget, s.store_none) == (2, 4, False)
    monkeypatch.setenv("CAREKV_PREFILL_RESIDUAL_KIND", "v")
    s = care_kv.resolve_store_knobs(c, 0)
    assert (s.k_budget, s.v_budget) == (0, 4)
    c = care_kv.CacheConfig(num_layers=1, group_size=32, store_budget_ratio=0.0)
    assert care_kv.resolve_store_knobs(c, 0).store_none


def test_layer_budget_multiplier_mean_one():
    import care_kv
    c = care_kv.CacheConfig(num_layers=22, group_size=32, budget_policy="u_shaped")
    m = [care_kv.layer_budget_multiplier(c, l) for l in range(22)]
    assert abs(sum(m) / 22 - 1.0) < 1e-12 and m[0] > 1.5 and m[11] < 0.6


def test_env_overrides(monkeypatch):
    import care_kv
    monkeypatch.setenv("CAREKV_BASE_BITS", "3")
    monkeypatch.setenv("CAREKV_SCALE_QUANT", "int8")
    monkeypatch.setenv("CAREKV_PACKED_BASE", "1")
    monkeypatch.setenv("CAREKV_LAYER_SENSITIVITY", "1.5,1.0")
    kw = care_kv.apply_carekv_env_overrides({})
    assert kw == dict(base_bits=3, scale_quant="int8", packed_base=True, layer_sensitivity=[1.5, 1.0])


def test_read_knobs(monkeypatch):
    import care_kv
    monkeypatch.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    monkeypatch.setenv("CAREKV_KSCORE_LIVE", "1")
    monkeypatch.setenv("CAREKV_SCORE_NORMALIZE", "1")
    c = care_kv.CacheConfig(num_layers=1, group_size=32, read_budget_mode="absolute", read_abs_k=128,
                            read_abs_v=128, route_policy="joint")
    r = care_kv.resolve_read_knobs(c, 0)
    assert (r.k_exact, r.kscore_live, r.normalize, r.joint, r.abs_k, r.abs_v, r.budget_ratio) == \
        (True, True, True, True, 128, 128, False)


def test_bench_rejects_multi_gpu():
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0 and "one GPU" in r.stderr


def test_adapter_interface_and_limits():
    """CAREKVAdapter keeps the reference constructor and reporting surface
    (baselines/carekv_adapter.py:23-263); unbuilt options raise."""
    from care_kv import CAREKVAdapter
    a = CAREKVAdapter(sk=2, sv=4, rk=2, rv=2, bits=3)
    assert a.name == "CAREKV_fixed_SK2SV4_RK2RV2"
    env = a.env()
    assert env["CAREKV_PREFILL_MODE"] == "carekv_stored" and env["CAREKV_STORE_ABS_V"] == "4"
    m = a.estimate_memory(2048, num_layers=22, hkv=4, head_dim=64)
    fp16 = 22 * 2 * 2048 * 4 * 64 * 2 / 2**20
    assert abs(m["base_memory_MB"] - round(fp16 * 3 / 16, 4)) < 1e-3
    assert a.effective_budgets()["effective_read_budget"] == "fixed RK=2 RV=2"
    with pytest.raises(NotImplementedError):
        CAREKVAdapter(base_quantizer="rotatekv_style")
    assert CAREKVAdapter(base_quantizer="kivi_style", bits=2).env()["CAREKV_BASE_QUANTIZER"] == "kivi_style"
    ad = CAREKVAdapter(mode="adaptive", rel_threshold=0.25, max_rk=4, max_rv=6)
    assert ad.name == "CAREKV_adaptive_rel0.25"
    e = ad.env()
    assert (e["CAREKV_READ_BUDGET_MODE"], e["CAREKV_READ_ABS_K"], e["CAREKV_READ_ABS_V"],
            e["CAREKV_READ_RELATIVE_THRESHOLD"]) == ("adaptive_score", "4", "6", "0.25")


def test_prefill_mode_resolution(monkeypatch):
    """_resolve_prefill_mode (layer.py:129-140)."""
    from care_kv.layer import resolve_prefill_mode
    for raw, want in (("fp", "fp"), ("quant", "base_quant"), ("int", "base_quant"), ("carekv", "carekv_eval"),
                      ("carekv_stored", "carekv_stored")):
        monkeypatch.setenv("CAREKV_PREFILL_MODE", raw)
        assert resolve_prefill_mode() == want
    monkeypatch.setenv("CAREKV_PREFILL_MODE", "bogus")
    with pytest.raises(ValueError):
        resolve_prefill_mode()


def test_prefill_correct_rejects_bad_rows():
    """carekv_prefill_correct_workspace_bytes validates the prompt rows and
    the read knobs on the host (no device call): rows outside the prompt, a
    prompt longer than the arena and correction off are refused with -1; a
    valid request sizes the workspace, with the sketch proxy (the router of
    correction_impl=cached) larger by its records and per-wave maxima."""
    import ctypes as C
    _lib = _ensure_built()
    lib = _lib.load()
    a = _lib.Arena(n_seq=2, n_kv_heads=2, max_pages=8, head_dim=64, base_bits=3, page_size=16, group_size=32,
                   k_channel_group=32, v_token_block=4, sketch_dim=32, scale_mode=1, residual_bits=4, n_slots=64)
    dp = _lib.DecodeParams(n_heads=8, correction=1, k_cap=2, v_cap=4, split_pages=16, lambda_k=1.0, lambda_v=1.0)

    def ws(**kw):
        p = dict(seq=0, n_tokens=100, row_begin=0, n_rows=100, k_hat=1, v_hat=1, lse=1)
        p.update(kw)
        return lib.carekv_prefill_correct_workspace_bytes(C.byref(a), C.byref(dp), C.byref(_lib.PrefillCorrParams(**p)))

    assert ws() > 0
    assert ws(row_begin=60, n_rows=41) == -1      # past the prompt
    assert ws(n_tokens=16 * 8 + 1, n_rows=1) == -1  # more pages than the arena row
    assert ws(seq=2) == -1                         # no such sequence slot
    assert ws(k_hat=0) == -1                       # missing K_hat
    live = ws()
    dp.k_proxy = 1
    assert ws() > live                             # the router's proxy records and logit maxima
    dp.k_proxy, dp.correction = 0, 0
    assert ws() == -1                              # the pass is the correction


def test_padding_mask_runs():
    """CAREKVLayer._key_runs: causal-only masks (boolean, additive, (T, T))
    need no split; a left- or right-padded sequence anywhere in the batch
    gets its run of real rows from the keys its last row sees (boolean
    (B, 1, T, S) masks as HF's sdpa path builds them, additive masks with
    -inf or the dtype's lowest value, (B, S) keep-masks); holes and score
    biases are refused."""
    import torch
    _ensure_built()
    from care_kv.layer import CAREKVLayer
    runs = CAREKVLayer._key_runs
    B, T = 3, 6
    causal = torch.tril(torch.ones(T, T, dtype=torch.bool))[None, None].expand(B, 1, T, T).clone()
    assert runs(causal, B, T) is None
    assert runs(torch.tril(torch.ones(T, T, dtype=torch.bool)), B, T) is None
    padded = causal.clone()
    padded[0, :, :, :2] = False                    # sequence 0 left-padded by two tokens
    padded[2, :, :, 4:] = False                    # sequence 2 right-padded by two
    assert runs(padded, B, T) == [(2, 6), (0, 6), (0, 4)]
    add = torch.zeros(B, 1, T, T, dtype=torch.float16)
    add.masked_fill_(~causal, torch.finfo(torch.float16).min)
    assert runs(add, B, T) is None
    add[1, :, :, 0] = float("-inf")                # only sequence 1 padded
    assert runs(add, B, T) == [(0, 6), (1, 6), (0, 6)]
    add[1, :, :, :] = float("-inf")                # an all-pad sequence: an empty run
    assert runs(add, B, T) == [(0, 6), (0, 0), (0, 6)]
    keep = torch.tensor([[1, 1, 1, 1], [0, 1, 1, 1]])
    assert runs(keep, 2, 3) is None                # the last 3 of 4 keys are real
    assert runs(keep, 2, 4) == [(0, 4), (1, 4)]
    holed = causal.clone()
    holed[1, :, :, 3] = False
    with pytest.raises(NotImplementedError):
        runs(holed, B, T)
    bias = torch.zeros(B, 1, T, T)
    bias[0, :, :, 1] = -0.5                        # a score bias, not a mask
    with pytest.raises(NotImplementedError):
        runs(bias, B, T)
    with pytest.raises(NotImplementedError):
        runs(torch.zeros(B, 1, T - 1, T - 1, dtype=torch.bool), B, T)


def test_patched_model_makes_a_carekv_hf_cache(monkeypatch):
    """patch_llama_model on transformers 5.x: generate's default cache and the
    decoder's own cache (use_cache, no cache given) are CAREKVHFCache, whose
    layers count the rows HF reads; a cache the caller passes is kept.  Run
    on the CPU with CAREKV_RETURN=original (HF's attention behind the patch),
    which exercises the cache plumbing without the HIP library."""
    import torch
    import care_kv
    transformers = pytest.importorskip("transformers")
    if int(transformers.__version__.split(".")[0]) < 5:
        pytest.skip("CAREKVHFCache is built for transformers 5.x")
    from transformers import DynamicCache, LlamaConfig, LlamaForCausalLM
    monkeypatch.setenv("CAREKV_RETURN", "original")
    torch.manual_seed(0)
    c = LlamaConfig(hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                    num_key_value_heads=2, vocab_size=100, max_position_embeddings=128)
    model = LlamaForCausalLM(c).eval()
    cfg = care_kv.CacheConfig(num_layers=2, num_heads=4, num_kv_heads=2, head_dim=16, max_pages=8)
    care_kv.patch_llama_model(model, cfg)
    ids = torch.randint(0, 100, (2, 9))
    with torch.no_grad():
        out = model.generate(ids, max_new_tokens=4, do_sample=False, return_dict_in_generate=True,
                             pad_token_id=0)
        pkv = out.past_key_values
        assert isinstance(pkv, care_kv.CAREKVHFCache)
        assert [pkv.get_seq_length(i) for i in range(2)] == [12, 12]   # 9 prompt rows + 3 fed back
        assert pkv.get_mask_sizes(1, 0) == (13, 0)
        mine = DynamicCache()
        out = model.generate(ids, max_new_tokens=2, do_sample=False, return_dict_in_generate=True,
                             pad_token_id=0, past_key_values=mine)
        assert out.past_key_values is mine
        r = model(ids, use_cache=True)
        assert isinstance(r.past_key_values, care_kv.CAREKVHFCache) and r.past_key_values.get_seq_length() == 9
        assert model(ids, use_cache=False).past_key_values is None
    with pytest.raises(NotImplementedError):
        pkv.crop(-1)


def test_prefill_eval_knobs_match_reference(monkeypatch):
    """carekv_eval knobs (layer.py:375-393): defaults, the read budget ratio
    as the ratio's default, errors on unknown kinds; the entry point refuses
    rows past its LDS score buffer before any launch."""
    import ctypes as C
    from care_kv import prefill
    _lib = _ensure_built()
    for k in ("CAREKV_PREFILL_RESIDUAL_RATIO", "CAREKV_PREFILL_MIN_RESIDUALS", "CAREKV_PREFILL_RESIDUAL_KIND",
              "CAREKV_V_SCORE", "CAREKV_SCORE_NORMALIZE", "CAREKV_K_CORRECTION_SCALE"):
        monkeypatch.delenv(k, raising=False)
    assert prefill.eval_knobs(0.07) == dict(ratio=0.07, min_residuals=1, kind="both", v_score="output_aware",
                                            normalize=False, k_corr_scale=0.1)
    monkeypatch.setenv("CAREKV_PREFILL_RESIDUAL_KIND", "V")
    monkeypatch.setenv("CAREKV_SCORE_NORMALIZE", "1")
    monkeypatch.setenv("CAREKV_PREFILL_RESIDUAL_RATIO", "0.2")
    kn = prefill.eval_knobs(0.07)
    assert (kn["kind"], kn["normalize"], kn["ratio"]) == ("v", True, 0.2)
    monkeypatch.setenv("CAREKV_PREFILL_RESIDUAL_KIND", "kv")
    with pytest.raises(ValueError):
        prefill.eval_knobs(0.0)
    monkeypatch.setenv("CAREKV_PREFILL_RESIDUAL_KIND", "both")
    monkeypatch.setenv("CAREKV_V_SCORE", "l2")
    with pytest.raises(ValueError):
        prefill.eval_knobs(0.0)
    lib = _lib.load()
    pp = _lib.PrefillEvalParams(batch=1, n_heads=2, n_kv_heads=2, seq_len=8193, head_dim=64, ratio=0.1,
                                min_residuals=1, kind=0, v_score_norm=0, normalize=0, k_corr_scale=0.1)
    fake = [C.c_void_p(4096)] * 7  # never dereferenced: the checks fail first
    assert lib.carekv_prefill_eval(pp, *fake, None, None) != 0
    assert b"seq_len" in lib.carekv_last_error()
    pp.seq_len, pp.n_kv_heads = 100, 3
    assert lib.carekv_prefill_eval(pp, *fake, None, None) != 0


def test_to_device_host_fallback_copies():
    """cache.to_device: on a host device a plain copy (the pinned,
    non-blocking path needs a GPU); dtype and values survive, and the result
    does not alias the source array (the append reuses its host arrays)."""
    import numpy as np
    import torch
    from care_kv.cache import to_device
    for dt, view in ((np.int32, True), (np.int64, True), (np.int32, False), (np.int64, False)):
        a = np.arange(12, dtype=dt).reshape(3, 4)
        if view:
            a = a[:, ::2]  # a non-contiguous view
        t = to_device(a, torch.device("cpu"))
        assert t.dtype == torch.from_numpy(a.copy()).dtype and t.is_contiguous()
        assert np.array_equal(t.numpy(), a)
        a[...] = -1
        assert not np.array_equal(t.numpy(), a)
