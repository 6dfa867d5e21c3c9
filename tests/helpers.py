"""Shared helpers for the parity tests (not collected by pytest)."""
from __future__ import annotations

import math
import os

import numpy as np

from oracle import quant as Q
from oracle.attention import decode_attention as oracle_decode
from oracle.cache import OCache, OCfg
from oracle.check import (compare_selection, decode_diag, oracle_candidates, oracle_selection,  # noqa: F401
                          output_errors, ties_explain)
from oracle.store import decode_append, write_pages_for_kv_head

F16, F32 = np.float16, np.float32
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# decode golden cases written by tests/golden/make_golden.py
DECODE_CASES = {
    "c1": dict(Hq=32, Hkv=4, D=64, store=dict(store_budget_mode="ratio", store_budget_ratio=0.03), k_mode="exact"),
    "c1_tight": dict(Hq=32, Hkv=4, D=64, store=dict(store_budget_mode="ratio", store_budget_ratio=0.03), k_mode="exact"),
    "gqa4_d128": dict(Hq=8, Hkv=2, D=128, store=dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4),
                      k_mode="exact"),
    "mha_d128_linear": dict(Hq=2, Hkv=2, D=128, store=dict(store_budget_mode="ratio", store_budget_ratio=0.03),
                            k_mode="linear"),
    # the sketch-proxy K score (CAREKV_KSCORE_LIVE=0)
    "c1_proxy": dict(Hq=32, Hkv=4, D=64, store=dict(store_budget_mode="ratio", store_budget_ratio=0.03),
                     k_mode="exact", live=False, score_rtol=1e-3, tie_eps=2e-3),
    "gqa4_d128_proxy": dict(Hq=8, Hkv=2, D=128, store=dict(store_budget_mode="absolute", store_abs_k=2,
                                                           store_abs_v=4), k_mode="exact", live=False,
                           score_rtol=1e-3, tie_eps=2e-3),
    # KIVI-style INT2 base in the fp16 side buffer (base_quantizer=kivi_style)
    # (the K score sums ||dS * A(1-A)|| over wider-spread logits than the
    # uniform INT3 cases: fp32 order differences reach 3e-5 relative)
    "c1_kivi": dict(Hq=32, Hkv=4, D=64, store=dict(store_budget_mode="ratio", store_budget_ratio=0.03),
                    k_mode="exact", base_quantizer="kivi_style", base_bits=2, score_rtol=1e-4),
    "gqa4_d128_kivi": dict(Hq=8, Hkv=2, D=128, store=dict(store_budget_mode="absolute", store_abs_k=2,
                                                          store_abs_v=4), k_mode="exact",
                           base_quantizer="kivi_style", base_bits=2, score_rtol=1e-4),
}

# prefill (carekv_stored, vectorized correction) golden cases
PREFILL_CASES = {
    "gqa8_d64": dict(Hq=16, Hkv=2, D=64, store=dict(store_budget_mode="ratio", store_budget_ratio=0.03),
                     k_mode="exact", policy="joint"),
    "gqa4_d128": dict(Hq=8, Hkv=2, D=128, store=dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4),
                      k_mode="exact", policy="separate"),
    "mha_d128_linear": dict(Hq=2, Hkv=2, D=128, store=dict(store_budget_mode="ratio", store_budget_ratio=0.03),
                            k_mode="linear", policy="joint"),
}


def prefill_cfg_kwargs(g, spec):
    T = int(g["T"])
    return dict(num_layers=1, num_heads=spec["Hq"], num_kv_heads=spec["Hkv"], head_dim=spec["D"], page_size=16,
                max_pages=T // 16 + 4, base_bits=3, group_size=32, k_channel_group=32, v_token_block=4,
                sketch_dim=32, read_budget_mode="absolute", read_abs_k=int(g["read_k"]),
                read_abs_v=int(g["read_v"]), route_policy=spec["policy"], **spec["store"])


def build_oracle_prefill(g, name):
    """Oracle cache of a prefill golden case and the page writer's K_hat / V_hat."""
    spec = PREFILL_CASES[name]
    c = OCache(OCfg(**prefill_cfg_kwargs(g, spec)))
    T = int(g["T"])
    kh, vh = [], []
    for h in range(spec["Hkv"]):
        a, b = write_pages_for_kv_head(c, 0, h, g["K"][h, :T], g["V"][h, :T], token_start_abs=0, sink_tokens=4)
        kh.append(a)
        vh.append(b)
    return c, spec, np.stack(kh), np.stack(vh)


PAPER_ENV = dict(CAREKV_STORE_POLICY="residual_kind_aware", CAREKV_PREFILL_RESIDUAL_KIND="both",
                 CAREKV_KSCORE_LIVE="1", CAREKV_SCORE_NORMALIZE="1", CAREKV_K_CORRECTION_SCALE="0.1")


def load_golden(name):
    return dict(np.load(os.path.join(GOLDEN, name), allow_pickle=False))


def case_cfg_kwargs(g, spec):
    T = int(g["T"])
    return dict(num_layers=1, num_heads=spec["Hq"], num_kv_heads=spec["Hkv"], head_dim=spec["D"], page_size=16,
                max_pages=max(T // 16 + 4, 400), base_bits=spec.get("base_bits", 3), group_size=32,
                k_channel_group=32, v_token_block=4, sketch_dim=32, read_budget_mode="absolute",
                read_abs_k=int(g["read_k"]), read_abs_v=int(g["read_v"]), route_policy="joint",
                base_quantizer=spec.get("base_quantizer", "uniform"), **spec["store"])


def build_oracle_case(g, name):
    spec = DECODE_CASES[name]
    c = OCache(OCfg(**case_cfg_kwargs(g, spec)))
    T, n_app = int(g["T"]), int(g["n_append"])
    for h in range(spec["Hkv"]):
        write_pages_for_kv_head(c, 0, h, g["K"][h, :T], g["V"][h, :T], token_start_abs=0, sink_tokens=4)
    for t in range(T, T + n_app):
        decode_append(c, 0, g["K"][:, t], g["V"][:, t])
    return c, spec


# prefill carekv_eval golden cases (tests/golden/make_golden.py:golden_prefill_eval)
EVAL_CASES = {
    "eval_gqa4_d64": dict(Hq=8, Hkv=2, D=64),
    "eval_mha_d128_k": dict(Hq=2, Hkv=2, D=128),
    "eval_gqa2_d128_v": dict(Hq=4, Hkv=2, D=128),
}


def eval_knobs(g):
    """prefill_eval knobs of a carekv_eval golden (the env it was written under)."""
    return dict(ratio=float(g["carekv_prefill_residual_ratio"]),
                min_residuals=int(g["carekv_prefill_min_residuals"]),
                kind=str(g["carekv_prefill_residual_kind"]), v_score=str(g["carekv_v_score"]),
                normalize=str(g["carekv_score_normalize"]) == "1",
                k_corr_scale=float(g["carekv_k_correction_scale"]))


def eval_hats(g, spec):
    """The page writer's K_hat / V_hat of a carekv_eval golden's prompt."""
    T = int(g["T"])
    c = OCache(OCfg(num_layers=1, num_heads=spec["Hq"], num_kv_heads=spec["Hkv"], head_dim=spec["D"], page_size=16,
                    max_pages=T // 16 + 4, base_bits=3, group_size=32, k_channel_group=32, v_token_block=4,
                    sketch_dim=32, store_budget_mode="ratio", store_budget_ratio=0.03))
    kh, vh = [], []
    for h in range(spec["Hkv"]):
        a, b = write_pages_for_kv_head(c, 0, h, g["K"][h, :T], g["V"][h, :T], token_start_abs=0, sink_tokens=4)
        kh.append(a)
        vh.append(b)
    return np.stack(kh), np.stack(vh)


def oracle_cache_arrays(c, layer=0):
    """An oracle cache's layer as the arrays of a store golden (the keys
    tests/golden/make_golden.py writes from the reference's cache): codes,
    scales, masters, valid counts, slot payloads and scales, and per page the
    slot ids (-2 where the page has no metadata), errors and sketches."""
    cfg = c.cfg
    d = dict(K_codes=c.base_K_codes[layer], V_codes=c.base_V_codes[layer], K_scale=c.base_K_scale[layer],
             V_scale=c.base_V_scale[layer], valid=c.valid_tokens[layer])
    if c.base_K_scale_master is not None:
        d["K_master"] = c.base_K_scale_master[layer]
        d["V_master"] = c.base_V_scale_master[layer]
    nk, nv = c.next_k_slot, c.next_v_slot
    d.update(k_res=c.k_residual_buf[:nk], k_res_scale=c.k_residual_scale[:nk], v_res=c.v_residual_buf[:nv],
             v_res_scale=c.v_residual_scale[:nv])
    H, P = c.valid_tokens.shape[1], c.valid_tokens.shape[2]
    ncg, nvb = cfg.head_dim // cfg.k_channel_group, math.ceil(cfg.page_size / cfg.v_token_block)
    ks = np.full((H, P, ncg), -2, np.int32)
    vs = np.full((H, P, nvb), -2, np.int32)
    ke = np.zeros((H, P, ncg), F16)
    ve = np.zeros((H, P, nvb), F16)
    sk = np.zeros((H, P, ncg, cfg.sketch_dim), F16)
    for h in range(H):
        for p in range(P):
            m = c.meta_table[layer][h][p]
            if m is None:
                continue
            ks[h, p], vs[h, p] = m.k_residual_slots, m.v_residual_slots
            ke[h, p], ve[h, p], sk[h, p] = m.k_error_norm, m.v_error_norm, m.k_sketch
    d.update(k_slots=ks, v_slots=vs, k_err=ke, v_err=ve, k_sketch=sk)
    return d
