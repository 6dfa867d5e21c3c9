"""Write golden input/output vectors from the reference implementation.

Run once in the build container (the reference is mounted read-only at
/root/reference; it never travels to the GPU box):

    python tests/golden/make_golden.py

Only the functions that no closed form, committed fixture or invariant pins
are exercised here (see the oracle package docstring):
  * ``CAREKVLayer._write_pages_for_kv_head`` -> ``CAREKVCache.write_base`` +
    ``ResidualStoreManager.process_page`` (fp16 chain, int8 scales, slots)
  * ``CAREKVCache.append_to_page`` / ``read_base_concat`` (int8 scales,
    decode-opened page)
  * ``vectorized_joint_correction`` under the comb+ex knobs and the
    reference test fixture's kind x policy x normalise grid.
Outputs are small ``.npz`` files next to this script.
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("CAREKV_REFERENCE", "/root/reference")


def _import_reference():
    root = "/tmp/carekv_ref_pkg"
    pkg = os.path.join(root, "CARE_KV")
    os.makedirs(pkg, exist_ok=True)
    open(os.path.join(pkg, "__init__.py"), "a").close()
    link = os.path.join(pkg, "care_kv")
    if not os.path.islink(link):
        os.symlink(REF, link)
    sys.path.insert(0, root)
    import CARE_KV.care_kv as ck  # noqa: F401
    return ck


def _set_env(**kw):
    for k, v in kw.items():
        os.environ[k] = str(v)


def _gen_kv(seed, n_kvh, T, D, outlier_ch=4, outlier_mult=8.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    K = torch.randn(n_kvh, T, D, generator=g)
    V = torch.randn(n_kvh, T, D, generator=g)
    for h in range(n_kvh):
        ch = torch.randperm(D, generator=g)[:outlier_ch]
        K[h][:, ch] *= outlier_mult
    return K.half(), V.half()


def _cache_arrays(cache, L=0):
    d = dict(
        K_codes=cache.base_K_codes[L].numpy(), V_codes=cache.base_V_codes[L].numpy(),
        K_scale=cache.base_K_scale[L].numpy(), V_scale=cache.base_V_scale[L].numpy(),
        valid=cache.valid_tokens[L].numpy(),
    )
    if getattr(cache, "base_K_hat_fp16", None) is not None:  # side-buffer base (KIVI)
        d["K_hat"] = cache.base_K_hat_fp16[L].numpy()
        d["V_hat"] = cache.base_V_hat_fp16[L].numpy()
    if cache.base_K_scale_master is not None:
        d["K_master"] = cache.base_K_scale_master[L].numpy()
        d["V_master"] = cache.base_V_scale_master[L].numpy()
    nk = cache.k_residual_buf.shape[0] - len(cache._k_slot_free)
    nv = cache.v_residual_buf.shape[0] - len(cache._v_slot_free)
    d["k_res"] = cache.k_residual_buf[:nk].numpy()
    d["k_res_scale"] = cache.k_residual_scale[:nk].numpy()
    d["v_res"] = cache.v_residual_buf[:nv].numpy()
    d["v_res_scale"] = cache.v_residual_scale[:nv].numpy()
    Hkv, P = cache.valid_tokens.shape[1], cache.valid_tokens.shape[2]
    cfg = cache.cfg
    ncg = cfg.head_dim // cfg.k_channel_group
    nvb = math.ceil(cfg.page_size / cfg.v_token_block)
    ks = np.full((Hkv, P, ncg), -2, np.int32)
    vs = np.full((Hkv, P, nvb), -2, np.int32)
    ke = np.zeros((Hkv, P, ncg), np.float16)
    ve = np.zeros((Hkv, P, nvb), np.float16)
    sk = np.zeros((Hkv, P, ncg, cfg.sketch_dim), np.float16)
    for h in range(Hkv):
        for p in range(P):
            m = cache.meta_table[L][h][p]
            if m is None:
                continue
            ks[h, p] = m.k_residual_slots
            vs[h, p] = m.v_residual_slots
            ke[h, p] = m.k_error_norm.numpy()
            ve[h, p] = m.v_error_norm.numpy()
            sk[h, p] = m.k_sketch.numpy()
    d.update(k_slots=ks, v_slots=vs, k_err=ke, v_err=ve, k_sketch=sk)
    return d


def _make_layer(ck, cfg):
    D, Hq, Hkv = cfg.head_dim, cfg.num_heads, cfg.num_kv_heads
    md = Hq * D
    W = torch.zeros(md, md)
    return ck.CAREKVLayer(cfg, 0, W, torch.zeros(Hkv * D, md), torch.zeros(Hkv * D, md), W)


def golden_store(ck):
    """Prefill page writes + store (fp16 chain) at D=128 / page 16 / g 32."""
    out = {}
    for tag, kw in (("abs", dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4)),
                    ("ratio", dict(store_budget_mode="ratio", store_budget_ratio=0.03))):
        _set_env(CAREKV_STORE_POLICY="residual_kind_aware", CAREKV_PREFILL_RESIDUAL_KIND="both")
        cfg = ck.CacheConfig(num_layers=1, num_heads=2, num_kv_heads=2, head_dim=128, page_size=16,
                             max_pages=8, base_bits=3, group_size=32, k_channel_group=32,
                             v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8", **kw)
        cache = ck.CAREKVCache(cfg, torch.device("cpu"))
        layer = _make_layer(ck, cfg)
        K, V = _gen_kv(11, 2, 40, 128)
        for h in range(2):
            layer._write_pages_for_kv_head(cache, h, K[h], V[h], token_start_abs=0, sink_tokens=4)
        d = _cache_arrays(cache)
        out.update({f"{tag}_{k}": v for k, v in d.items()})
    out["K"] = K.numpy()
    out["V"] = V.numpy()
    np.savez_compressed(os.path.join(HERE, "store_d128.npz"), **out)


def golden_append(ck):
    """int8-scale append into a prefill page and into a decode-opened page."""
    cfg = ck.CacheConfig(num_layers=1, num_heads=1, num_kv_heads=1, head_dim=64, page_size=16,
                         max_pages=4, base_bits=3, group_size=32, packed_base=True,
                         scale_quant="int8", store_budget_mode="absolute")
    cache = ck.CAREKVCache(cfg, torch.device("cpu"))
    qc = ck.QuantConfig(bits=3, group_size=32)
    g = torch.Generator().manual_seed(5)
    X = (torch.randn(2, 16 + 3 + 2, 64, generator=g) * 1.5).half()
    page = torch.cat([X[:, :10], torch.zeros(2, 6, 64).half()], 1)
    Kc, Ks = ck.quantize(page[0], qc)
    Vc, Vs = ck.quantize(page[1], qc)
    p0 = cache.alloc_page(0, 0)
    cache.write_base(0, 0, p0, Kc, Ks, Vc, Vs, num_valid=10)
    rows = []
    for i in range(10, 16):
        kc, ks = ck.quantize(X[0, i:i + 1], qc)
        vc, vs = ck.quantize(X[1, i:i + 1], qc)
        cache.append_to_page(0, 0, p0, kc[0], ks[0], vc[0], vs[0])
    p1 = cache.alloc_page(0, 0)
    cache.valid_tokens[0, 0, p1] = 0
    for i in range(16, 21):
        kc, ks = ck.quantize(X[0, i:i + 1], qc)
        vc, vs = ck.quantize(X[1, i:i + 1], qc)
        cache.append_to_page(0, 0, p1, kc[0], ks[0], vc[0], vs[0])
    Kc2, Ks2, Vc2, Vs2, lens = cache.read_base_concat(0, 0, [p0, p1])
    d = _cache_arrays(cache)
    d.update(X=X.numpy(), read_Kc=Kc2.numpy(), read_Ks=Ks2.numpy(), read_Vc=Vc2.numpy(),
             read_Vs=Vs2.numpy(), read_lens=np.array(lens))
    np.savez_compressed(os.path.join(HERE, "append_d64.npz"), **d)


def _selector_layer(ck, cfg):
    """CAREKVLayer whose projections pick q/k/v out of hidden = [q; k; v] and
    whose W_O returns the attention output unchanged (exact in fp16)."""
    D, Hq, Hkv = cfg.head_dim, cfg.num_heads, cfg.num_kv_heads
    nq, nk = Hq * D, Hkv * D
    md = nq + 2 * nk
    eye = torch.eye(md, dtype=torch.float16)
    W_Q, W_K, W_V = eye[:nq], eye[nq:nq + nk], eye[nq + nk:]
    W_O = eye[:, :nq].contiguous()
    return ck.CAREKVLayer(cfg, 0, W_Q.contiguous(), W_K.contiguous(), W_V.contiguous(), W_O)


def _decode_case(ck, name, *, Hq, Hkv, D, T, seed, outlier_mult, store, read_k, read_v,
                 n_append=0, k_mode="exact", kscore_live=True, base_quantizer="uniform", base_bits=3):
    from CARE_KV.care_kv.attention import vectorized_joint_correction, set_chunk_recorder
    _set_env(CAREKV_STORE_POLICY="residual_kind_aware", CAREKV_PREFILL_RESIDUAL_KIND="both",
             CAREKV_K_CORRECTION_MODE=k_mode, CAREKV_KSCORE_LIVE="1" if kscore_live else "0",
             CAREKV_SCORE_NORMALIZE="1", CAREKV_DEBUG_STATS="0")
    cfg = ck.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                         max_pages=max(T // 16 + 4, 400), base_bits=base_bits, group_size=32, k_channel_group=32,
                         v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8",
                         read_budget_ratio=0.0, read_budget_mode="absolute", read_abs_k=read_k,
                         read_abs_v=read_v, route_policy="joint", base_quantizer=base_quantizer, **store)
    cache = ck.CAREKVCache(cfg, torch.device("cpu"))
    layer = _selector_layer(ck, cfg)
    K, V = _gen_kv(seed, Hkv, T + n_append, D, outlier_mult=outlier_mult)
    qg = torch.Generator().manual_seed(seed + 100)
    Qall = torch.randn(n_append + 1, Hq, D, generator=qg).half()
    for h in range(Hkv):
        layer._write_pages_for_kv_head(cache, h, K[h, :T], V[h, :T], token_start_abs=0, sink_tokens=4)
    # decode steps through the reference's own decode_step (append, store on
    # page fill, base attention; read_budget_ratio=0 gates its correction off)
    dec_out = None
    for i, t in enumerate(range(T, T + n_append)):
        hidden = torch.cat([Qall[i].reshape(-1), K[:, t].reshape(-1), V[:, t].reshape(-1)])[None]
        dec_out = layer.decode_step(cache, hidden)
    Qh = Qall[max(n_append - 1, 0)] if n_append > 0 else Qall[0]
    rec = []
    set_chunk_recorder(rec)
    grp = Hq // Hkv
    O_out = torch.zeros(Hq, D)
    per = {}
    sf = 1.0 / math.sqrt(D)
    for h in range(Hkv):
        pids = cache.all_page_ids(0, h)
        if base_quantizer == "uniform":
            Kc, Ks, Vc, Vs, _ = cache.read_base_concat(0, h, pids)
            N = Kc.shape[0]
            Kb = ck.dequantize(Kc, Ks, (N, D), layer.base_qcfg).float()
            Vb = ck.dequantize(Vc, Vs, (N, D), layer.base_qcfg).float()
        else:  # the fp16 side buffer (attention.py:997-1008)
            Kh, Vh, _ = cache.read_base_hat_concat(0, h, pids)
            Kb, Vb = Kh.float(), Vh.float()
        heads = list(range(h * grp, (h + 1) * grp))
        S = torch.stack([(Kb @ Qh[i].float()) * sf for i in heads])
        A = torch.softmax(S, dim=1)
        O = torch.stack([(A[j].unsqueeze(-1) * Vb).sum(0) for j in range(len(heads))])
        n0 = len(rec)
        delta = vectorized_joint_correction(cache, cfg, layer.router, 0, h, pids,
                                            Q_q=Qh[heads].float(), S=S, A=A, V_base=Vb, O_base=O,
                                            kind="both", k_corr_scale=0.1, score_normalize=True)
        O_out[heads] = (O + delta.float())
        r = rec[n0] if len(rec) > n0 else {}
        for key in ("score_K", "score_V", "sel_k", "sel_v"):
            v = r.get(key)
            if v is not None:
                per[f"h{h}_{key}"] = v.numpy()
        per[f"h{h}_O_base"] = O.numpy()
        per[f"h{h}_delta"] = delta.float().numpy()
    set_chunk_recorder(None)
    d = _cache_arrays(cache)
    d.update(per)
    d.update(K=K.numpy(), V=V.numpy(), Qall=Qall.numpy(), Q=Qh.numpy(), O=O_out.half().numpy(),
             T=np.array(T), n_append=np.array(n_append), read_k=np.array(read_k), read_v=np.array(read_v))
    if dec_out is not None:
        d["decode_step_out"] = dec_out[0, :Hq * D].reshape(Hq, D).numpy()
    np.savez_compressed(os.path.join(HERE, f"decode_{name}.npz"), **d)


def golden_decode(ck):
    ratio3 = dict(store_budget_mode="ratio", store_budget_ratio=0.03)
    # config 1 (TinyLlama shape): B=1, 32q/4kv, D=64, 512 ctx, top-64 read, 4 outlier ch x8
    _decode_case(ck, "c1", Hq=32, Hkv=4, D=64, T=512, seed=1, outlier_mult=8.0,
                 store=ratio3, read_k=32, read_v=32)
    # same shape, a tight read budget so the joint top-k actually selects
    _decode_case(ck, "c1_tight", Hq=32, Hkv=4, D=64, T=512, seed=1, outlier_mult=8.0,
                 store=ratio3, read_k=4, read_v=4)
    # GQA 4, D=128 slice with a partial page, paper store budget SK=2 SV=4, and decode appends
    _decode_case(ck, "gqa4_d128", Hq=8, Hkv=2, D=128, T=1000, seed=3, outlier_mult=10.0,
                 store=dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4),
                 read_k=16, read_v=16, n_append=27)
    # MHA slice (c2 shape per head), linear K mode for coverage
    _decode_case(ck, "mha_d128_linear", Hq=2, Hkv=2, D=128, T=512, seed=2, outlier_mult=6.0,
                 store=ratio3, read_k=8, read_v=8, k_mode="linear")


def golden_decode_kivi(ck):
    """KIVI-style base (per-channel K over the whole prompt, per-token V,
    fp16 side buffer; kivi_helpers.py:35-59, cache.py:797-865) under the
    same comb+ex correction, INT2 as in config 3."""
    ratio3 = dict(store_budget_mode="ratio", store_budget_ratio=0.03)
    _decode_case(ck, "c1_kivi", Hq=32, Hkv=4, D=64, T=512, seed=1, outlier_mult=8.0,
                 store=ratio3, read_k=32, read_v=32, base_quantizer="kivi_style", base_bits=2)
    _decode_case(ck, "gqa4_d128_kivi", Hq=8, Hkv=2, D=128, T=1000, seed=3, outlier_mult=10.0,
                 store=dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4),
                 read_k=16, read_v=16, n_append=27, base_quantizer="kivi_style", base_bits=2)


def golden_decode_proxy(ck):
    """The sketch-proxy K score (CAREKV_KSCORE_LIVE=0, attention.py:718-725)
    under the same comb+ex knobs otherwise."""
    ratio3 = dict(store_budget_mode="ratio", store_budget_ratio=0.03)
    _decode_case(ck, "c1_proxy", Hq=32, Hkv=4, D=64, T=512, seed=1, outlier_mult=8.0,
                 store=ratio3, read_k=4, read_v=4, kscore_live=False)
    _decode_case(ck, "gqa4_d128_proxy", Hq=8, Hkv=2, D=128, T=1000, seed=3, outlier_mult=10.0,
                 store=dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4),
                 read_k=16, read_v=16, n_append=27, kscore_live=False)


def _prefill_case(ck, name, *, Hq, Hkv, D, T, seed, outlier_mult, store, read_k, read_v, k_mode="exact",
                  policy="joint", base_bits=3, impl="vectorized", kscore_live=1):
    """CAREKVLayer.prefill in carekv_stored mode (layer.py:643-840) with the
    vectorized correction over all kv_group x T queries of a kv head
    (layer.py:538-557): the causal base attention over the prefill's own
    K_hat / V_hat, then vectorized_joint_correction with the fp16 attention
    weights.  Also the base_quant output of the same prompt (fresh cache)."""
    from CARE_KV.care_kv.attention import set_chunk_recorder
    env = dict(CAREKV_STORE_POLICY="residual_kind_aware", CAREKV_PREFILL_RESIDUAL_KIND="both",
               CAREKV_K_CORRECTION_MODE=k_mode, CAREKV_KSCORE_LIVE=str(kscore_live), CAREKV_SCORE_NORMALIZE="1",
               CAREKV_DEBUG_STATS="0", CAREKV_CORRECTION_IMPL=impl)
    _set_env(**env)
    K, V = _gen_kv(seed, Hkv, T, D, outlier_mult=outlier_mult)
    qg = torch.Generator().manual_seed(seed + 200)
    Q = torch.randn(T, Hq, D, generator=qg).half()
    hidden = torch.cat([Q.reshape(T, -1), K.permute(1, 0, 2).reshape(T, -1), V.permute(1, 0, 2).reshape(T, -1)], 1)
    out = {}
    for mode in ("base_quant", "carekv_stored"):
        _set_env(CAREKV_PREFILL_MODE=mode)
        cfg = ck.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                             max_pages=T // 16 + 4, base_bits=base_bits, group_size=32, k_channel_group=32,
                             v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8",
                             read_budget_ratio=0.0, read_budget_mode="absolute", read_abs_k=read_k,
                             read_abs_v=read_v, route_policy=policy, correction_impl=impl, **store)
        cache = ck.CAREKVCache(cfg, torch.device("cpu"))
        layer = _selector_layer(ck, cfg)
        rec = []
        set_chunk_recorder(rec)
        o = layer.prefill(cache, hidden)
        set_chunk_recorder(None)
        out[mode] = o[:, :Hq * D].reshape(T, Hq, D).numpy()
        if mode == "carekv_stored":
            # per kv head, the query chunks' records in query order (the
            # assembled record of a chunked call carries no scores)
            for h in range(Hkv):
                parts = sorted((r for r in rec if r["kv_head"] == h and r.get("q_offset", 0) != -1),
                               key=lambda r: r.get("q_offset", 0))
                for key in ("score_K", "score_V", "sel_k", "sel_v"):
                    vs = [r.get(key) for r in parts]
                    if vs and all(v is not None for v in vs):
                        out[f"h{h}_{key}"] = torch.cat(vs, 0).numpy()
    d = _cache_arrays(cache)
    d.update({k: v for k, v in out.items() if k.startswith("h")})
    d.update(K=K.numpy(), V=V.numpy(), Q=Q.numpy(), O=out["carekv_stored"], O_base=out["base_quant"],
             T=np.array(T), n_append=np.array(0), read_k=np.array(read_k), read_v=np.array(read_v))
    _set_env(CAREKV_PREFILL_MODE="fp", CAREKV_CORRECTION_IMPL="cached", CAREKV_KSCORE_LIVE="1")
    np.savez_compressed(os.path.join(HERE, f"prefill_{name}.npz"), **d)


def golden_prefill(ck):
    ratio3 = dict(store_budget_mode="ratio", store_budget_ratio=0.03)
    # TinyLlama head shape (GQA 8, D=64), a partial last page, tight joint read
    _prefill_case(ck, "gqa8_d64", Hq=16, Hkv=2, D=64, T=200, seed=21, outlier_mult=8.0, store=ratio3,
                  read_k=4, read_v=4)
    # GQA 4, D=128, paper store budget SK=2 SV=4, separate policy
    _prefill_case(ck, "gqa4_d128", Hq=8, Hkv=2, D=128, T=150, seed=22, outlier_mult=10.0,
                  store=dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4), read_k=6, read_v=6,
                  policy="separate")
    # MHA, linear K mode
    _prefill_case(ck, "mha_d128_linear", Hq=2, Hkv=2, D=128, T=120, seed=23, outlier_mult=6.0, store=ratio3,
                  read_k=3, read_v=3, k_mode="linear")


def golden_prefill_cached(ck):
    """CAREKVLayer.prefill in carekv_stored mode with correction_impl="cached"
    (the CAREKVAdapter default): the per-(head, row) apply_slot_corrections
    loop over ResidualRouter.route (layer.py:573-640, attention.py:208-374,
    residual_router.py:88-452).  The router has no query-aware K score, so
    CAREKV_KSCORE_LIVE=1 must give the same output as 0 (the second case)."""
    ratio3 = dict(store_budget_mode="ratio", store_budget_ratio=0.03)
    _prefill_case(ck, "cached_gqa4_d64", Hq=8, Hkv=2, D=64, T=100, seed=31, outlier_mult=8.0,
                  store=dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4), read_k=4, read_v=4,
                  k_mode="exact", policy="joint", impl="cached", kscore_live=0)
    _prefill_case(ck, "cached_mha_d128_linear", Hq=2, Hkv=2, D=128, T=90, seed=32, outlier_mult=6.0, store=ratio3,
                  read_k=3, read_v=3, k_mode="linear", policy="separate", impl="cached", kscore_live=1)


def golden_prefill_eval(ck):
    """CAREKVLayer.prefill in carekv_eval mode (layer.py:792-806, 363-456):
    the causal base attention over the prefill's K_hat / V_hat, then the
    per-(head, row) top-k correction from the full in-memory residuals.
    Three knob sets: both kinds normalised with the output-aware V score,
    the K kind alone with a larger residual ratio, and the V kind alone
    (output-aware score, min_residuals 2)."""
    cases = (("eval_gqa4_d64", dict(Hq=8, Hkv=2, D=64, T=90, seed=41, outlier_mult=8.0),
              dict(CAREKV_PREFILL_RESIDUAL_RATIO="0.05", CAREKV_PREFILL_MIN_RESIDUALS="1",
                   CAREKV_PREFILL_RESIDUAL_KIND="both", CAREKV_V_SCORE="output_aware", CAREKV_SCORE_NORMALIZE="1",
                   CAREKV_K_CORRECTION_SCALE="0.1")),
             ("eval_mha_d128_k", dict(Hq=2, Hkv=2, D=128, T=70, seed=42, outlier_mult=10.0),
              dict(CAREKV_PREFILL_RESIDUAL_RATIO="0.1", CAREKV_PREFILL_MIN_RESIDUALS="2",
                   CAREKV_PREFILL_RESIDUAL_KIND="k", CAREKV_V_SCORE="norm", CAREKV_SCORE_NORMALIZE="0",
                   CAREKV_K_CORRECTION_SCALE="0.3")),
             ("eval_gqa2_d128_v", dict(Hq=4, Hkv=2, D=128, T=80, seed=43, outlier_mult=8.0),
              dict(CAREKV_PREFILL_RESIDUAL_RATIO="0.04", CAREKV_PREFILL_MIN_RESIDUALS="2",
                   CAREKV_PREFILL_RESIDUAL_KIND="v", CAREKV_V_SCORE="output_aware", CAREKV_SCORE_NORMALIZE="0",
                   CAREKV_K_CORRECTION_SCALE="0.1")))
    only = os.environ.get("CAREKV_GOLDEN_EVAL_CASES")
    if only:
        cases = tuple(c for c in cases if c[0] in only.split(","))
    for name, shape, env in cases:
        Hq, Hkv, D, T = shape["Hq"], shape["Hkv"], shape["D"], shape["T"]
        _set_env(CAREKV_PREFILL_MODE="carekv_eval", CAREKV_DEBUG_STATS="0", **env)
        K, V = _gen_kv(shape["seed"], Hkv, T, D, outlier_mult=shape["outlier_mult"])
        Q = torch.randn(T, Hq, D, generator=torch.Generator().manual_seed(shape["seed"] + 200)).half()
        hidden = torch.cat([Q.reshape(T, -1), K.permute(1, 0, 2).reshape(T, -1), V.permute(1, 0, 2).reshape(T, -1)], 1)
        cfg = ck.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                             max_pages=T // 16 + 4, base_bits=3, group_size=32, k_channel_group=32, v_token_block=4,
                             sketch_dim=32, packed_base=True, scale_quant="int8", read_budget_ratio=0.0,
                             store_budget_mode="ratio", store_budget_ratio=0.03)
        cache = ck.CAREKVCache(cfg, torch.device("cpu"))
        o = _selector_layer(ck, cfg).prefill(cache, hidden)
        d = dict(K=K.numpy(), V=V.numpy(), Q=Q.numpy(), O=o[:, :Hq * D].reshape(T, Hq, D).numpy(), T=np.array(T),
                 **{k.lower(): np.array(v) for k, v in env.items()})
        np.savez_compressed(os.path.join(HERE, f"prefill_{name}.npz"), **d)
    _set_env(CAREKV_PREFILL_MODE="fp", CAREKV_PREFILL_RESIDUAL_KIND="both", CAREKV_SCORE_NORMALIZE="1",
             CAREKV_K_CORRECTION_SCALE="0.1")


def _decode_step_case(ck, name, *, Hq, Hkv, D, T, n_append, seed, outlier_mult, store, read_k, read_v, k_mode,
                      policy):
    """The reference's decode_step with its correction gate open
    (read_budget_ratio > 0, attention.py:1025): every step appends the token
    (store on page fill with K_orig = K_hat) and runs CAREKVMultiHeadAttention
    with apply_slot_corrections over ResidualRouter.route (the sketch-proxy
    selector; the router reads no CAREKV_KSCORE_LIVE) under the absolute
    read budgets.  Every step's output is kept."""
    _set_env(CAREKV_STORE_POLICY="residual_kind_aware", CAREKV_PREFILL_RESIDUAL_KIND="both",
             CAREKV_K_CORRECTION_MODE=k_mode, CAREKV_KSCORE_LIVE="1", CAREKV_SCORE_NORMALIZE="1",
             CAREKV_K_CORRECTION_SCALE="0.1", CAREKV_DEBUG_STATS="0")
    cfg = ck.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                         max_pages=T // 16 + n_append // 16 + 4, base_bits=3, group_size=32, k_channel_group=32,
                         v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8",
                         read_budget_ratio=0.03, read_budget_mode="absolute", read_abs_k=read_k,
                         read_abs_v=read_v, route_policy=policy, **store)
    cache = ck.CAREKVCache(cfg, torch.device("cpu"))
    layer = _selector_layer(ck, cfg)
    K, V = _gen_kv(seed, Hkv, T + n_append, D, outlier_mult=outlier_mult)
    Qall = torch.randn(n_append, Hq, D, generator=torch.Generator().manual_seed(seed + 300)).half()
    for h in range(Hkv):
        layer._write_pages_for_kv_head(cache, h, K[h, :T], V[h, :T], token_start_abs=0, sink_tokens=4)
    outs = []
    for i, t in enumerate(range(T, T + n_append)):
        hidden = torch.cat([Qall[i].reshape(-1), K[:, t].reshape(-1), V[:, t].reshape(-1)])[None]
        outs.append(layer.decode_step(cache, hidden)[0, :Hq * D].reshape(Hq, D))
    d = _cache_arrays(cache)
    d.update(K=K.numpy(), V=V.numpy(), Qall=Qall.numpy(), outs=torch.stack(outs).numpy(), T=np.array(T),
             n_append=np.array(n_append), read_k=np.array(read_k), read_v=np.array(read_v))
    np.savez_compressed(os.path.join(HERE, f"decode_step_{name}.npz"), **d)


def golden_decode_step(ck):
    # GQA 4, D=128: the prompt's partial page fills and a decode-opened page
    # follows (zero master); joint read of 6 + 6 slots, exact K correction
    _decode_step_case(ck, "gqa4_d128", Hq=8, Hkv=2, D=128, T=250, n_append=24, seed=41, outlier_mult=10.0,
                      store=dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4), read_k=6,
                      read_v=6, k_mode="exact", policy="joint")
    # GQA 8, D=64 (TinyLlama heads), separate policy, linear K correction
    _decode_step_case(ck, "gqa8_d64_linear", Hq=16, Hkv=2, D=64, T=120, n_append=12, seed=42, outlier_mult=8.0,
                      store=dict(store_budget_mode="ratio", store_budget_ratio=0.03), read_k=5, read_v=5,
                      k_mode="linear", policy="separate")


ROUTE_VARIANTS = [  # (route_policy, adaptive_score (rel, abs, min_keep) or None)
    ("joint", None), ("separate", None), ("k_first", None), ("adaptive", None),
    ("joint", (0.5, 0.0, 0)), ("separate", (0.0, 1.5, 3)), ("k_first", (0.8, 0.0, 2)), ("adaptive", (0.3, 0.9, 0)),
]


def golden_route(ck):
    """ResidualRouter.route (residual_router.py:88-452) selections per query
    under every route_policy and the adaptive_score thresholds, with the raw
    candidate scores of vectorized_joint_correction (KSCORE_LIVE=0, the same
    score formulas at sensitivity 1) and the attention rows they came from."""
    from CARE_KV.care_kv.attention import vectorized_joint_correction, set_chunk_recorder
    _set_env(CAREKV_STORE_POLICY="residual_kind_aware", CAREKV_PREFILL_RESIDUAL_KIND="both",
             CAREKV_K_CORRECTION_MODE="exact", CAREKV_KSCORE_LIVE="0", CAREKV_SCORE_NORMALIZE="1",
             CAREKV_DEBUG_STATS="0")
    Hq, Hkv, D, T = 8, 2, 64, 300
    cfg = ck.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16, max_pages=64,
                         base_bits=3, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                         packed_base=True, scale_quant="int8", read_budget_ratio=0.0, read_budget_mode="absolute",
                         read_abs_k=6, read_abs_v=6, route_policy="joint", store_budget_mode="absolute",
                         store_abs_k=2, store_abs_v=2)
    cache = ck.CAREKVCache(cfg, torch.device("cpu"))
    layer = _selector_layer(ck, cfg)
    K, V = _gen_kv(7, Hkv, T, D, outlier_mult=8.0)
    Qh = torch.randn(Hq, D, generator=torch.Generator().manual_seed(8)).half()
    for h in range(Hkv):
        layer._write_pages_for_kv_head(cache, h, K[h], V[h], token_start_abs=0, sink_tokens=4)
    out = {}
    grp = Hq // Hkv
    sf = 1.0 / math.sqrt(D)
    for h in range(Hkv):
        pids = cache.all_page_ids(0, h)
        Kc, Ks, Vc, Vs, _ = cache.read_base_concat(0, h, pids)  # the uniform base
        N = Kc.shape[0]
        Kb = ck.dequantize(Kc, Ks, (N, D), layer.base_qcfg).float()
        Vb = ck.dequantize(Vc, Vs, (N, D), layer.base_qcfg).float()
        heads = list(range(h * grp, (h + 1) * grp))
        S = torch.stack([(Kb @ Qh[i].float()) * sf for i in heads])
        A = torch.softmax(S, dim=1)
        O = torch.stack([(A[j].unsqueeze(-1) * Vb).sum(0) for j in range(grp)])
        rec = []
        set_chunk_recorder(rec)
        vectorized_joint_correction(cache, cfg, layer.router, 0, h, pids, Q_q=Qh[heads].float(), S=S, A=A,
                                    V_base=Vb, O_base=O, kind="both", k_corr_scale=0.1, score_normalize=True)
        set_chunk_recorder(None)
        out[f"h{h}_score_K"] = rec[0]["score_K"].numpy()
        out[f"h{h}_score_V"] = rec[0]["score_V"].numpy()
        out[f"h{h}_A"] = A.numpy()
        kc, vc = [], []
        for pid in pids:
            m = cache.meta_table[0][h][pid]
            nv = int(cache.valid_tokens[0, h, pid].item())
            if nv == 0 or m is None:
                continue
            kc += [(pid, cg) for cg, sl in enumerate(m.k_residual_slots) if sl >= 0]
            vc += [(pid, vb) for vb, sl in enumerate(m.v_residual_slots) if sl >= 0 and vb * 4 < nv]
        out[f"h{h}_kcand"] = np.array(kc, np.int32).reshape(-1, 2)
        out[f"h{h}_vcand"] = np.array(vc, np.int32).reshape(-1, 2)
        for vi, (pol, asc) in enumerate(ROUTE_VARIANTS):
            cfg.route_policy = pol
            cfg.read_budget_mode = "adaptive_score" if asc else "absolute"
            if asc:
                cfg.read_relative_threshold, cfg.read_absolute_threshold, cfg.read_min_keep = asc
            for j, qh in enumerate(heads):
                ks, vs = layer.router.route(cache=cache, kv_head=h, page_ids=pids, q=Qh[qh].float(), s_base=S[j],
                                            a_base=A[j], O_base=O[j], V_base_full=Vb, kind="both",
                                            score_normalize=True)
                out[f"h{h}_v{vi}_q{j}_k"] = np.array([(p, c) for p, c, _ in ks], np.int32).reshape(-1, 2)
                out[f"h{h}_v{vi}_q{j}_v"] = np.array([(p, b) for p, b, _ in vs], np.int32).reshape(-1, 2)
        cfg.route_policy, cfg.read_budget_mode = "joint", "absolute"
    out["budgets"] = np.array([6, 6], np.int32)
    np.savez_compressed(os.path.join(HERE, "route_d64.npz"), **out)


def golden_reference_fixture(ck):
    """The reference's own test fixture (tests/test_vectorized_carekv.py:30-58):
    D=32, page 8, g 8, kcg 16, vtb 4, sketch 4, SK=SV=2, fp32 inputs."""
    from CARE_KV.care_kv.attention import vectorized_joint_correction, set_chunk_recorder
    out = {}
    torch.manual_seed(0)
    Ks = [torch.randn(8, 32) for _ in range(4)]
    Vs = [torch.randn(8, 32) for _ in range(4)]
    qs = torch.randn(3, 32)
    for pol in ("joint", "separate"):
        for live in (0, 1):
            for mode in ("linear", "exact"):
                _set_env(CAREKV_KSCORE_LIVE=live, CAREKV_K_CORRECTION_MODE=mode,
                         CAREKV_STORE_POLICY="residual_kind_aware", CAREKV_PREFILL_RESIDUAL_KIND="both")
                cfg = ck.CacheConfig(num_layers=1, num_heads=3, num_kv_heads=1, head_dim=32, page_size=8,
                                     max_pages=4, base_bits=3, group_size=8, k_channel_group=16,
                                     v_token_block=4, store_budget_mode="absolute",
                                     read_budget_mode="absolute", store_abs_k=2, store_abs_v=2,
                                     read_abs_k=2, read_abs_v=2, sketch_dim=4, route_policy=pol)
                cache = ck.CAREKVCache(cfg, torch.device("cpu"))
                sm = ck.ResidualStoreManager(cfg, 0, torch.device("cpu"))
                router = ck.ResidualRouter(cfg, 0, torch.device("cpu"))
                qc = ck.QuantConfig(bits=3, group_size=8)
                for p in range(4):
                    Kc, Ksc, _, _ = ck.quantize_and_residual(Ks[p], qc)
                    Vc, Vsc, _, _ = ck.quantize_and_residual(Vs[p], qc)
                    pid = cache.alloc_page(0, 0)
                    cache.write_base(0, 0, pid, Kc, Ksc, Vc, Vsc, num_valid=8)
                    sm.process_page(cache, 0, pid, Ks[p], Vs[p], Kc, Ksc, Vc, Vsc,
                                    token_start=p * 8, num_valid=8)
                pids = list(range(4))
                Kc, Ksc, Vc, Vsc, _ = cache.read_base_concat(0, 0, pids)
                N = Kc.shape[0]
                Kb = ck.dequantize(Kc, Ksc, (N, 32), qc).float()
                Vb = ck.dequantize(Vc, Vsc, (N, 32), qc).float()
                S = (qs @ Kb.T) / math.sqrt(32)
                A = torch.softmax(S, dim=1)
                O = A @ Vb
                for kind in ("both", "k", "v"):
                    for norm in (False, True):
                        rec = []
                        set_chunk_recorder(rec)
                        dlt = vectorized_joint_correction(cache, cfg, router, 0, 0, pids, Q_q=qs, S=S, A=A,
                                                          V_base=Vb, O_base=O, kind=kind, k_corr_scale=0.1,
                                                          score_normalize=norm)
                        set_chunk_recorder(None)
                        tag = f"{pol}_live{live}_{mode}_{kind}_n{int(norm)}"
                        out[f"{tag}_delta"] = dlt.numpy()
                        if rec:
                            for key in ("sel_k", "sel_v"):
                                if rec[0].get(key) is not None:
                                    out[f"{tag}_{key}"] = rec[0][key].numpy()
                if pol == "joint" and live == 0 and mode == "linear":
                    d = _cache_arrays(cache)
                    out.update({f"cache_{k}": v for k, v in d.items()})
    out["K"] = torch.stack(Ks).numpy()
    out["V"] = torch.stack(Vs).numpy()
    out["Q"] = qs.numpy()
    np.savez_compressed(os.path.join(HERE, "ref_fixture_d32.npz"), **out)


def golden_sketch(ck):
    from CARE_KV.care_kv.residual_store import get_sketch_proj
    np.save(os.path.join(HERE, "sketch_proj_32x32.npy"),
            get_sketch_proj(128, 32, 32, torch.device("cpu")).numpy())




def golden_activation_slices():
    """Slices of the reference-held TinyLlama activations (INT3, g=32, fp32
    chain; results/paper_eval_20260529_015053/figures/3d_data, produced by
    tools/make_before_after_3d_figures.py:227-279) used as a known-answer
    test of the fp32 quantizer.  Plain .npy data, loaded without pickle."""
    src = os.path.join(REF, "results/paper_eval_20260529_015053/figures/3d_data")
    out = {}
    for layer, rows in (("00", 64), ("21", 32)):
        for nm in ("k_fp", "k_hat", "v_fp", "v_hat"):
            a = np.load(os.path.join(src, f"layer{layer}_{nm}.npy"), allow_pickle=False)
            out[f"l{layer}_{nm}"] = a[:rows].astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "activations_3d_slices.npz"), **out)


PARTS = ("activations", "sketch", "store", "append", "decode", "decode_proxy", "decode_kivi", "prefill", "route",
         "fixture", "prefill_cached", "decode_step", "prefill_eval")

if __name__ == "__main__":
    # CAREKV_GOLDEN_PARTS=decode_proxy,... writes only those fixtures
    parts = [p for p in os.environ.get("CAREKV_GOLDEN_PARTS", ",".join(PARTS)).split(",") if p]
    if os.environ.get("CAREKV_GOLDEN_ONLY_ACTIVATIONS", "0") == "1":
        parts = ["activations"]
    torch.set_num_threads(1)
    if "activations" in parts:
        golden_activation_slices()
    if any(p != "activations" for p in parts):
        ck = _import_reference()
        fns = dict(sketch=golden_sketch, store=golden_store, append=golden_append, decode=golden_decode,
                   decode_proxy=golden_decode_proxy, decode_kivi=golden_decode_kivi, prefill=golden_prefill,
                   route=golden_route, fixture=golden_reference_fixture,
                   prefill_cached=golden_prefill_cached, decode_step=golden_decode_step,
                   prefill_eval=golden_prefill_eval)
        for p in parts:
            if p in fns:
                fns[p](ck)
    print("golden fixtures written to", HERE)
