"""Store-time residual candidates and selection (``residual_store.py:206-464``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np

from . import quant as Q
from .cache import OCache, OMeta, layer_budget_multiplier

F16, F32 = np.float16, np.float32


def sketch_proj(k_channel_group: int, sketch_dim: int):
    """``residual_store.py:206-214``: randn(kcg, sd, CPU generator seed 42)/sqrt(sd).

    torch's CPU normal generator is a library routine; the committed fixture
    ``tests/golden/sketch_proj_32x32.npy`` pins its values for (32, 32)."""
    import torch  # library routine only; the oracle itself is numpy
    gen = torch.Generator(device="cpu").manual_seed(42)
    P = torch.randn(k_channel_group, sketch_dim, generator=gen) / math.sqrt(sketch_dim)
    return P.numpy().astype(F32)


def _norm_rows(x):
    """fp32 L2 norm over the last axis."""
    x = np.asarray(x, dtype=F32)
    return np.sqrt((x * x).sum(axis=-1, dtype=F32), dtype=F32)


def process_page(cache: OCache, layer_id: int, kv_head: int, page_id: int,
                 K_orig, V_orig, K_codes, K_scale, V_codes, V_scale,
                 token_start: int, num_valid: int, is_recent=True, is_sink=False,
                 store_policy: str = "residual_kind_aware", residual_kind: str = "both",
                 min_per_kind: int = 1, k_frac: float = 1.0, v_frac: float = 1.0,
                 K_hat_override=None, V_hat_override=None, P=None, reuse_slots: bool = False) -> OMeta:
    """``ResidualStoreManager.process_page`` (``residual_store.py:239-464``)
    with the default (no-op) selector-variant / position-policy knobs.

    ``reuse_slots=True`` (no reference counterpart; the streaming fill
    store): the slot ids of the page's earlier metadata (a prompt's partial
    last page), ascending, go to the first selected candidates of their kind
    before new ids are allocated; ids no longer needed stay unused.  The reference overwrites the metadata
    and orphans them (``residual_store.py:463``)."""
    cfg = cache.cfg
    K_orig = np.asarray(K_orig)
    V_orig = np.asarray(V_orig)
    T, D = K_orig.shape
    sens = float(cfg.layer_sensitivity[layer_id])
    if K_hat_override is not None and V_hat_override is not None:
        K_hat = np.asarray(K_hat_override).astype(K_orig.dtype)
        V_hat = np.asarray(V_hat_override).astype(V_orig.dtype)
    else:
        K_hat = Q.dequantize(K_codes, K_scale, cfg.group_size)
        V_hat = Q.dequantize(V_codes, V_scale, cfg.group_size)
    # (K_orig - K_hat) in the input dtype, then .float()   (residual_store.py:279-280)
    R_K = Q._rt(K_orig.astype(F32) - K_hat.astype(F32), K_orig.dtype).astype(F32)
    R_V = Q._rt(V_orig.astype(F32) - V_hat.astype(F32), V_orig.dtype).astype(F32)
    if num_valid < T:
        R_K[num_valid:] = 0
        R_V[num_valid:] = 0
    struct_prior = 1.0
    if is_recent:
        struct_prior *= 1.5
    if is_sink:
        struct_prior *= 2.0
    if P is None:
        P = sketch_proj(cfg.k_channel_group, cfg.sketch_dim)

    kcg, vtb = cfg.k_channel_group, cfg.v_token_block
    num_cg = D // kcg
    k_cands, k_errs = [], []
    for cg in range(num_cg):
        c0, c1 = cg * kcg, (cg + 1) * kcg
        if num_valid > 0:
            blk = R_K[:num_valid, c0:c1]
            err = float(F32(_norm_rows(blk).mean(dtype=F32)))
            rk_mean = blk.mean(axis=0, dtype=F32)
        else:
            err = 0.0
            rk_mean = np.zeros(kcg, F32)
        k_errs.append(err)
        sketch = (rk_mean @ P).astype(F32).astype(F16)
        prior = err * sens * struct_prior
        packed, scale = Q.pack_residual(R_K[:, c0:c1], cfg.residual_bits)
        k_cands.append(dict(kind="K", idx=cg, payload=packed, scale=scale, sketch=sketch, prior=prior))

    num_vb = math.ceil(cfg.page_size / vtb)
    v_cands, v_errs = [], []
    for vb in range(num_vb):
        t0 = vb * vtb
        t1v = min(t0 + vtb, num_valid)
        err = float(F32(_norm_rows(R_V[t0:t1v]).mean(dtype=F32))) if t1v > t0 else 0.0
        v_errs.append(err)
        prior = err * sens * struct_prior
        blk = R_V[t0:t0 + vtb]
        if blk.shape[0] < vtb:
            blk = np.concatenate([blk, np.zeros((vtb - blk.shape[0], D), F32)])
        packed, scale = Q.pack_residual(blk, cfg.residual_bits)
        v_cands.append(dict(kind="V", idx=vb, payload=packed, scale=scale, sketch=None, prior=prior))

    k_scored = sorted([c for c in k_cands if c["prior"] > 0], key=lambda c: c["prior"], reverse=True)
    v_scored = sorted([c for c in v_cands if c["prior"] > 0], key=lambda c: c["prior"], reverse=True)
    use_k = use_v = True
    if store_policy == "residual_kind_aware":
        use_k = residual_kind != "v"
        use_v = residual_kind != "k"
    lm = layer_budget_multiplier(cfg, layer_id)
    if cfg.store_budget_mode == "absolute":
        k_budget = int(round(max(0, int(cfg.store_abs_k)) * lm)) if use_k else 0
        v_budget = int(round(max(0, int(cfg.store_abs_v)) * lm)) if use_v else 0
        joint_budget = k_budget + v_budget
    else:
        def _res(o, fb):
            return fb if (o is None or o < 0) else o
        rk = _res(cfg.store_budget_ratio_k, cfg.store_budget_ratio) * k_frac * lm
        rv = _res(cfg.store_budget_ratio_v, cfg.store_budget_ratio) * v_frac * lm
        k_total = max(1, len(k_cands))
        v_total = max(1, len(v_cands))
        k_budget = max(min_per_kind, int(k_total * rk)) if (use_k and rk > 0) else 0
        v_budget = max(min_per_kind, int(v_total * rv)) if (use_v and rv > 0) else 0
        joint_budget = max(1, int((k_total + v_total) * cfg.store_budget_ratio * lm))
    if (cfg.store_budget_ratio <= 0 and cfg.store_budget_mode != "absolute"
            and (cfg.store_budget_ratio_k or 0) <= 0 and (cfg.store_budget_ratio_v or 0) <= 0):
        selected = []
    elif store_policy == "joint":
        selected = sorted(k_scored + v_scored, key=lambda c: c["prior"], reverse=True)[:joint_budget]
    else:
        selected = k_scored[:k_budget] + v_scored[:v_budget]

    k_slots = [-1] * num_cg
    v_slots = [-1] * num_vb
    old = cache.meta_table[layer_id][kv_head][page_id] if reuse_slots else None
    reuse_k = sorted(x for x in old.k_residual_slots if x >= 0) if old is not None else []
    reuse_v = sorted(x for x in old.v_residual_slots if x >= 0) if old is not None else []
    for c in selected:
        if c["kind"] == "K":
            s = reuse_k.pop(0) if reuse_k else cache.alloc_k_slot()
            cache.write_k_residual(s, c["payload"], c["scale"])
            k_slots[c["idx"]] = s
        else:
            s = reuse_v.pop(0) if reuse_v else cache.alloc_v_slot()
            cache.write_v_residual(s, c["payload"], c["scale"])
            v_slots[c["idx"]] = s
    meta = OMeta(page_id=page_id, layer_id=layer_id, kv_head=kv_head, token_start=token_start,
                 num_tokens=num_valid, k_residual_slots=k_slots, v_residual_slots=v_slots,
                 k_error_norm=np.array(k_errs, dtype=F32).astype(F16),
                 v_error_norm=np.array(v_errs, dtype=F32).astype(F16),
                 k_sketch=np.stack([c["sketch"] for c in k_cands]),
                 prior_score=float(sum(c["prior"] for c in selected)))
    cache.meta_table[layer_id][kv_head][page_id] = meta
    return meta


def write_pages_for_kv_head(cache: OCache, layer_id: int, kv_h: int, K_kv, V_kv,
                            token_start_abs: int = 0, sink_tokens: int = 4, P=None, **store_kw):
    """``layer.py:204-334``: pad, quantize, write, store.  Returns the prompt's
    (K_hat, V_hat) over its valid rows as the reference's page writer does
    (layer.py:331-334): half(code * fp16 group scale) for the uniform base
    (the pages keep the int8-requantised scales), the KIVI quant-dequant for
    the side-buffer bases."""
    cfg = cache.cfg
    K_kv = np.asarray(K_kv)
    V_kv = np.asarray(V_kv)
    T, D = K_kv.shape
    ps = cfg.page_size
    num_pages = math.ceil(T / ps)
    if cfg.side_buffer:
        # layer.py:226-299: K_hat / V_hat over the whole prompt, pages of the
        # fp16 side buffer, residuals against them (kivi_style / kvquant_style
        # post-RoPE: per-channel K, per-token V)
        assert cfg.base_quantizer in ("kivi_style", "kvquant_style"), cfg.base_quantizer
        kb, vb = cfg.kivi_bits()
        Kh_seq = Q.kivi_qdq(K_kv, kb, per_channel=True).astype(K_kv.dtype)
        Vh_seq = Q.kivi_qdq(V_kv, vb, per_channel=False).astype(V_kv.dtype)
        for p in range(num_pages):
            t0, t1 = p * ps, min((p + 1) * ps, T)
            nv = t1 - t0
            pad = lambda a: np.concatenate([a, np.zeros((ps - nv, D), a.dtype)]) if nv < ps else a
            Kp, Vp, Khp, Vhp = pad(K_kv[t0:t1]), pad(V_kv[t0:t1]), pad(Kh_seq[t0:t1]), pad(Vh_seq[t0:t1])
            pid = cache.alloc_page(layer_id, kv_h)
            cache.write_base_kivi(layer_id, kv_h, pid, Khp, Vhp, num_valid=nv)
            process_page(cache, layer_id, kv_h, pid, Kp, Vp, None, None, None, None,
                         token_start=token_start_abs + t0, num_valid=nv, is_recent=p >= num_pages - 4,
                         is_sink=(token_start_abs + t0) < sink_tokens, K_hat_override=Khp, V_hat_override=Vhp,
                         P=P, **store_kw)
            if nv < ps:  # the open page's true rows, for a streaming fill store
                cache.open_rows[(layer_id, kv_h, pid)] = (Kp.copy(), Vp.copy())
        return Kh_seq, Vh_seq
    k_hat, v_hat = [], []
    for p in range(num_pages):
        t0, t1 = p * ps, min((p + 1) * ps, T)
        nv = t1 - t0
        Kp, Vp = K_kv[t0:t1], V_kv[t0:t1]
        if nv < ps:
            Kp = np.concatenate([Kp, np.zeros((ps - nv, D), K_kv.dtype)])
            Vp = np.concatenate([Vp, np.zeros((ps - nv, D), V_kv.dtype)])
        pid = cache.alloc_page(layer_id, kv_h)
        is_sink = (token_start_abs + t0) < sink_tokens
        is_recent = p >= num_pages - 4
        Kc, Ks = Q.quantize(Kp, cfg.base_bits, cfg.group_size)
        Vc, Vs = Q.quantize(Vp, cfg.base_bits, cfg.group_size)
        cache.write_base(layer_id, kv_h, pid, Kc, Ks, Vc, Vs, num_valid=nv)
        process_page(cache, layer_id, kv_h, pid, Kp, Vp, Kc, Ks, Vc, Vs,
                     token_start=token_start_abs + t0, num_valid=nv,
                     is_recent=is_recent, is_sink=is_sink, P=P, **store_kw)
        if nv < ps:  # the open page's true rows and fp16 group scales (streaming store, re-encoding append)
            cache.open_rows[(layer_id, kv_h, pid)] = (Kp.copy(), Vp.copy())
            cache.open_scales[(layer_id, kv_h, pid)] = (np.asarray(Ks, F16)[:nv].copy(), np.asarray(Vs, F16)[:nv].copy())
        k_hat.append(Q.dequantize(Kc, Ks, cfg.group_size).astype(K_kv.dtype)[:nv])
        v_hat.append(Q.dequantize(Vc, Vs, cfg.group_size).astype(V_kv.dtype)[:nv])
    return np.concatenate(k_hat), np.concatenate(v_hat)


def decode_append(cache: OCache, layer_id: int, k_rows, v_rows, streaming: bool = False, rescale: bool = False,
                  **store_kw):
    """Cache side of ``CAREKVLayer.decode_step`` (``layer.py:1001-1146``,
    uniform base quantizer): append one token per kv head into the open page
    (allocating one when full) and, when the append fills the page, run the
    store with K_orig = K_hat (zero residual, so the page gets metadata with no
    slots and a refilled partial prefill page loses its slots).

    ``streaming=True`` (no reference counterpart): the open
    page's true rows are kept (``cache.open_rows``, the prompt's partial last
    page included) and the fill store runs process_page on them against the
    page's own codes and read-back scales (the page's K_hat / V_hat rows for
    the side-buffer base), so decode-filled pages get residual slots.

    ``rescale=True`` (no reference counterpart; int8 page scales): instead of
    encoding the row's scales against the page's fixed master
    (``cache.py:689-695``, zero on a page the decode opened), the open page
    is re-encoded as ``write_base`` encodes its valid rows so far
    (``write_scale_page`` over their fp16 group scales, ``cache.py:592-604``),
    unless it holds stored residual slots (a prompt's partial last page: its
    slots are residuals against its rows as the prompt wrote them, so it
    keeps the fixed-master encoding until it fills).
    Together with ``streaming=True`` this is the decode path of a cache
    built with ``compat=False``; its fill store reuses the page's slot ids."""
    cfg = cache.cfg
    k_rows = np.asarray(k_rows)
    v_rows = np.asarray(v_rows)
    ps = cfg.page_size
    pos_abs = cache.total_valid_tokens(layer_id, 0)
    for h in range(cfg.num_kv_heads):
        pid = cache.get_open_page(layer_id, h)
        if pid is None:
            pid = cache.alloc_page(layer_id, h)
            cache.valid_tokens[layer_id, h, pid] = 0
        if streaming:
            kt, vt = cache.open_rows.setdefault(
                (layer_id, h, pid), (np.zeros((ps, cfg.head_dim), k_rows.dtype), np.zeros((ps, cfg.head_dim), v_rows.dtype)))
            off = int(cache.valid_tokens[layer_id, h, pid])
            kt[off], vt[off] = k_rows[h], v_rows[h]
        if cfg.side_buffer:
            # layer.py:1037-1075 (post-RoPE): the row quantised alone, K per
            # channel over T = 1, V per token; on fill K_orig = K_hat (:1089-1101)
            kb, vb = cfg.kivi_bits()
            kh = Q.kivi_qdq(k_rows[h:h + 1], kb, per_channel=True)[0]
            vh = Q.kivi_qdq(v_rows[h:h + 1], vb, per_channel=False)[0]
            cache.append_to_page_kivi(layer_id, h, pid, kh, vh)
            if int(cache.valid_tokens[layer_id, h, pid]) == ps:
                Kh = cache.base_K_hat_fp16[layer_id, h, pid].astype(k_rows.dtype)
                Vh = cache.base_V_hat_fp16[layer_id, h, pid].astype(v_rows.dtype)
                ts = pos_abs + 1 - ps
                Ko, Vo = cache.open_rows.pop((layer_id, h, pid)) if streaming else (Kh, Vh)
                process_page(cache, layer_id, h, pid, Ko, Vo, None, None, None, None, token_start=ts,
                             num_valid=ps, is_recent=True, is_sink=ts < 4, K_hat_override=Kh,
                             V_hat_override=Vh, reuse_slots=streaming, **store_kw)
            continue
        kc, ks = Q.quantize(k_rows[h:h + 1], cfg.base_bits, cfg.group_size)
        vc, vs = Q.quantize(v_rows[h:h + 1], cfg.base_bits, cfg.group_size)
        meta = cache.meta_table[layer_id][h][pid]
        has_slots = meta is not None and (any(x >= 0 for x in meta.k_residual_slots)
                                          or any(x >= 0 for x in meta.v_residual_slots))
        off = cache.append_to_page(layer_id, h, pid, kc[0], ks[0], vc[0], vs[0])
        if rescale and cfg.scale_quant == "int8" and not has_slots:
            G = cfg.head_dim // cfg.group_size
            oks, ovs = cache.open_scales.get((layer_id, h, pid), (np.zeros((0, G), F16), np.zeros((0, G), F16)))
            oks = np.concatenate([oks[:off], np.asarray(ks, F16)[:1]])
            ovs = np.concatenate([ovs[:off], np.asarray(vs, F16)[:1]])
            cache.open_scales[(layer_id, h, pid)] = (oks, ovs)
            for S, dst, mst in ((oks, cache.base_K_scale, cache.base_K_scale_master),
                                (ovs, cache.base_V_scale, cache.base_V_scale_master)):
                codes, master = Q.write_scale_page(S)
                dst[layer_id, h, pid, :off + 1] = codes
                mst[layer_id, h, pid] = master
            if off + 1 == ps:
                cache.open_scales.pop((layer_id, h, pid), None)
        if int(cache.valid_tokens[layer_id, h, pid]) == ps:
            Kc = cache.unpack_rows(cache.base_K_codes[layer_id, h, pid])
            Vc = cache.unpack_rows(cache.base_V_codes[layer_id, h, pid])
            Ks = cache.page_scales(layer_id, h, pid, "K")
            Vs = cache.page_scales(layer_id, h, pid, "V")
            Kh = Q.dequantize(Kc, Ks, cfg.group_size).astype(k_rows.dtype)
            Vh = Q.dequantize(Vc, Vs, cfg.group_size).astype(v_rows.dtype)
            ts = pos_abs + 1 - ps
            if streaming:  # the true rows instead of K_hat
                Kh, Vh = cache.open_rows.pop((layer_id, h, pid))
            process_page(cache, layer_id, h, pid, Kh, Vh, Kc, Ks, Vc, Vs, token_start=ts,
                         num_valid=ps, is_recent=True, is_sink=ts < 4, reuse_slots=streaming, **store_kw)
