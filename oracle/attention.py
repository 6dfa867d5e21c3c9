"""Decode attention and the batched joint correction (comb+ex selector).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``attention.py`` of the reference:
  * ``exact_softmax_correction``   -- attention.py:96-118
  * ``query_aware_kscore_slot``    -- attention.py:167-184
  * ``_build_v_slot_index``        -- attention.py:386-441
  * ``_build_k_slot_index``        -- attention.py:540-573
  * ``vectorized_joint_correction``-- attention.py:576-957 (default knobs:
    no prefilter, no chunking, no selector/position variants, raw_error V
    score, no K clamp/guard)
  * ``_resolve_read_budgets``      -- residual_router.py:37-76
  * ``route_selection``            -- the selection of ResidualRouter.route
    (residual_router.py:275-410): per-kind normalisation, the joint /
    separate / k_first / adaptive policies and the adaptive_score
    thresholds, on given per-query score rows
  * ``decode_attention``           -- attention.py:979-1077 with the
    correction call swapped for the batched joint correction over the GQA
    group's queries (per-query-row semantics, attention.py:830-875).
  * ``causal_attention_pure``      -- layer.py:935-972 (the prefill
    attention over dequantised K/V, attention_mask=None branch), with the
    GQA heads of layer.py:774-775 read in place.
  * ``prefill_eval``               -- layer.py:363-456, 792-806 (the
    carekv_eval prefill: token-level top-k over the full in-memory
    residuals).
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np

from . import quant as Q
from .cache import OCache, layer_budget_multiplier

F16, F32 = np.float16, np.float32
EPS = 1e-6


def softmax_rows(S):
    S = np.asarray(S, dtype=F32)
    m = S.max(axis=-1, keepdims=True)
    e = np.exp(S - m, dtype=F32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=F32)).astype(F32)


def exact_softmax_correction(A, ds, V_base, O_base, RV_full=None, sel_tok=None):
    """attention.py:96-118 (fp32)."""
    A = np.asarray(A, F32); ds = np.asarray(ds, F32)
    V_base = np.asarray(V_base, F32); O_base = np.asarray(O_base, F32)
    w = np.exp(ds - ds.max(axis=1, keepdims=True), dtype=F32)
    a_new = A * w
    a_new = a_new / np.maximum(a_new.sum(axis=1, keepdims=True, dtype=F32), F32(1e-30))
    O_new = a_new @ V_base
    if RV_full is not None and sel_tok is not None:
        O_new = O_new + (a_new * sel_tok.astype(F32)) @ np.asarray(RV_full, F32)
    return (O_new - O_base).astype(F32)


def query_aware_kscore_slot(Q_slot, dK_slot, A_slot, V_slot, head_dim):
    """attention.py:167-184: ||dS * A(1-A)||_tokens * ||V_slot||_F."""
    dS = (np.asarray(Q_slot, F32) @ np.asarray(dK_slot, F32).T) / F32(math.sqrt(max(head_dim, 1)))
    A_slot = np.asarray(A_slot, F32)
    sens = A_slot * (F32(1.0) - A_slot)
    kp = np.sqrt(((dS * sens) ** 2).sum(axis=1, dtype=F32), dtype=F32)
    vc = F32(np.sqrt((np.asarray(V_slot, F32) ** 2).sum(dtype=F32)))
    out = kp * vc
    out = np.nan_to_num(out, nan=0.0, posinf=0.0, neginf=0.0)
    return np.maximum(out, F32(0.0)).astype(F32)


def resolve_read_budgets(cfg, kind, total_k, total_v, layer_id=0):
    """residual_router.py:37-76."""
    lm = layer_budget_multiplier(cfg, layer_id)
    if cfg.read_budget_mode in ("absolute", "adaptive_score"):
        bk = int(round(max(0, int(cfg.read_abs_k)) * lm))
        bv = int(round(max(0, int(cfg.read_abs_v)) * lm))
    else:
        def _r(o, fb):
            return fb if (o is None or o < 0) else o
        rk = _r(cfg.read_budget_ratio_k, cfg.read_budget_ratio) * lm
        rv = _r(cfg.read_budget_ratio_v, cfg.read_budget_ratio) * lm
        bk = max(1, int(total_k * rk)) if rk > 0 and total_k > 0 else 0
        bv = max(1, int(total_v * rv)) if rv > 0 and total_v > 0 else 0
    if kind == "v":
        bk = 0
    elif kind == "k":
        bv = 0
    return min(bk, total_k), min(bv, total_v)


def build_v_slot_index(cache: OCache, layer_id, kv_head, page_ids, sens):
    """attention.py:386-441 (keeps the reference's cursor handling)."""
    cfg = cache.cfg
    vtb, D = cfg.v_token_block, cfg.head_dim
    resids, starts, lens, errs, ids = [], [], [], [], []
    cursor = 0
    for pid in page_ids:
        meta = cache.meta_table[layer_id][kv_head][pid]
        nv = int(cache.valid_tokens[layer_id, kv_head, pid])
        if nv == 0 or meta is None:
            continue
        for vb, slot in enumerate(meta.v_residual_slots):
            if slot < 0:
                continue
            t0 = vb * vtb
            t1 = min(t0 + vtb, nv)
            if t1 <= t0:
                continue
            r = Q.unpack_residual(cache.v_residual_buf[slot], cache.v_residual_scale[slot, 0],
                                  vtb * D, cfg.residual_bits).reshape(vtb, D)
            resids.append(r)
            starts.append(cursor + t0)
            lens.append(t1 - t0)
            errs.append(float(meta.v_error_norm[vb]) * sens)
            ids.append((pid, vb, slot))
        cursor += nv
    if not resids:
        return None
    return (np.stack(resids).astype(F32), np.array(starts, np.int64), np.array(lens, np.int64),
            np.array(errs, dtype=np.float64).astype(F32), ids)


def build_k_slot_index(cache: OCache, layer_id, kv_head, page_ids):
    """attention.py:540-573."""
    cfg = cache.cfg
    out = dict(R=[], cg=[], sketch=[], pstart=[], nvalid=[], ids=[])
    cursor = 0
    for pid in page_ids:
        meta = cache.meta_table[layer_id][kv_head][pid]
        nv = int(cache.valid_tokens[layer_id, kv_head, pid])
        if nv == 0 or meta is None:
            cursor += nv
            continue
        if meta.k_sketch is not None:
            for cg, slot in enumerate(meta.k_residual_slots):
                if slot < 0:
                    continue
                r = Q.unpack_residual(cache.k_residual_buf[slot], cache.k_residual_scale[slot, 0],
                                      cfg.page_size * cfg.k_channel_group,
                                      cfg.residual_bits).reshape(cfg.page_size, cfg.k_channel_group)
                out["R"].append(r[:nv].astype(F32))
                out["cg"].append(cg)
                out["sketch"].append(meta.k_sketch[cg].astype(F32))
                out["pstart"].append(cursor)
                out["nvalid"].append(nv)
                out["ids"].append((pid, cg, slot))
        cursor += nv
    return out


def route_selection(sK, sV, bk, bv, policy, kind, normalize, A_row=None, adaptive_score=False, rel_thr=0.0,
                    abs_thr=0.0, min_keep=0):
    """residual_router.py:275-410 for one query: sK / sV are the raw K / V
    candidate scores (None when that kind has no candidates), bk / bv the
    resolved budgets.  Python-float arithmetic and stable sorts as in the
    reference.  Returns boolean selection rows (None for an absent kind)."""
    kc = [] if sK is None else [(float(s), i) for i, s in enumerate(sK)]
    vc = [] if sV is None else [(float(s), i) for i, s in enumerate(sV)]
    selk = None if sK is None else np.zeros(len(kc), bool)
    selv = None if sV is None else np.zeros(len(vc), bool)
    if len(kc) + len(vc) == 0 or (bk == 0 and bv == 0):
        return selk, selv

    def _norm(c):
        if not c:
            return c
        mean = sum(abs(x[0]) for x in c) / len(c)
        sc = mean if mean > EPS else EPS
        return [(x[0] / sc, x[1]) for x in c]
    if normalize and kind == "both":
        kc, vc = _norm(kc), _norm(vc)
    desc = lambda c: sorted(c, key=lambda x: x[0], reverse=True)  # noqa: E731  stable
    if policy == "joint":
        mb = bk + bv if (bk > 0 and bv > 0) else max(bk, bv)
        allc = [("K",) + x for x in kc] + [("V",) + x for x in vc]
        sel = sorted(allc, key=lambda x: x[1], reverse=True)[:mb]
    elif policy == "k_first":
        kp = desc(kc)[:bk]
        rem = max(0, bk + bv - len(kp))
        vs = desc(vc)
        vp = []
        if vs and rem > 0:
            vmean = sum(x[0] for x in vs) / len(vs)
            vp = [x for x in vs if x[0] >= vmean][:rem]
        sel = [("K",) + x for x in kp] + [("V",) + x for x in vp]
    elif policy == "adaptive":
        total = bk + bv
        sel = []
        if total > 0:
            a = np.maximum(np.asarray(A_row, F32), F32(EPS))
            ent = float(-(a * np.log(a)).sum(dtype=F32))
            max_ent = math.log(max(a.size, 2))
            v_frac = max(0.0, min(1.0, ent / max_ent))
            v_alloc = max(0, int(round(total * v_frac)))
            k_alloc = max(0, total - v_alloc)
            sel = [("K",) + x for x in desc(kc)[:k_alloc]] + [("V",) + x for x in desc(vc)[:v_alloc]]
    else:
        sel = [("K",) + x for x in desc(kc)[:bk]] + [("V",) + x for x in desc(vc)[:bv]]
    if adaptive_score:
        def _filter(lst):
            if not lst:
                return lst
            top = float(abs(lst[0][1]))
            kept = [c for c in lst if (rel_thr <= 0 or abs(c[1]) >= rel_thr * top)
                    and (abs_thr <= 0 or abs(c[1]) >= abs_thr)]
            if min_keep > 0 and len(kept) < min_keep:
                kept = lst[:min(min_keep, len(lst))]
            return kept
        sk_ = sorted([c for c in sel if c[0] == "K"], key=lambda c: c[1], reverse=True)
        sv_ = sorted([c for c in sel if c[0] == "V"], key=lambda c: c[1], reverse=True)
        sel = _filter(sk_) + _filter(sv_)
    for c in sel:
        (selk if c[0] == "K" else selv)[c[2]] = True
    return selk, selv


def topk_lowest_index(scores, k):
    """Per-row top-k with ties resolved toward the lowest index."""
    order = np.argsort(-scores, axis=1, kind="stable")
    return order[:, :k]


def vectorized_joint_correction(cache: OCache, layer_id, kv_head, page_ids, Q_q, S, A, V_base, O_base,
                                kind="both", k_corr_scale=1.0, score_normalize=True,
                                kscore_live=True, k_mode="exact", lam_k=1.0, lam_v=1.0,
                                sketch_P=None, force_sel=None, diag: Optional[dict] = None):
    """attention.py:576-957 -> delta (Q, D) fp32.

    ``force_sel`` = (sel_k, sel_v) boolean masks replaces the top-k so a
    caller can recompute the delta under another implementation's selection
    (used to compare outputs across an epsilon-tie in the scores)."""
    cfg = cache.cfg
    Q_q = np.asarray(Q_q, F32); S = np.asarray(S, F32); A = np.asarray(A, F32)
    V_base = np.asarray(V_base, F32); O_base = np.asarray(O_base, F32)
    Qn, D = Q_q.shape
    N = A.shape[1]
    delta = np.zeros((Qn, D), F32)
    if diag is not None:
        diag.update(n_k=0, n_v=0, budget_k=0, budget_v=0)
    if N == 0:
        return delta
    sens = float(cfg.layer_sensitivity[layer_id])
    policy = cfg.route_policy
    v_idx = build_v_slot_index(cache, layer_id, kv_head, page_ids, sens)
    kx = build_k_slot_index(cache, layer_id, kv_head, page_ids)
    n_k = len(kx["R"])
    n_v = 0 if v_idx is None else v_idx[0].shape[0]
    want_k = kind in ("k", "both") and n_k > 0
    want_v = kind in ("v", "both") and n_v > 0
    if diag is not None:
        diag.update(n_k=n_k, n_v=n_v, k_ids=kx["ids"], v_ids=(v_idx[4] if v_idx else []))
    if not want_k and not want_v:
        return delta
    bk, bv = resolve_read_budgets(cfg, kind, n_k if want_k else 0, n_v if want_v else 0, layer_id)
    if diag is not None:
        diag.update(budget_k=bk, budget_v=bv)
    if bk == 0 and bv == 0:
        return delta

    kcg = cfg.k_channel_group
    # policies and thresholds only ResidualRouter.route has
    route_mode = policy in ("k_first", "adaptive") or cfg.read_budget_mode == "adaptive_score"
    score_K = None
    if want_k and (bk > 0 or route_mode):
        score_K = np.zeros((Qn, n_k), F32)
        need_proxy = not kscore_live
        if need_proxy:
            s_top = S.max(axis=1, keepdims=True)
            inv_margin = F32(1.0) / np.maximum(s_top - S, F32(EPS))
            vdiff = np.sqrt(((V_base[None] - O_base[:, None]) ** 2).sum(-1, dtype=F32), dtype=F32)
            if sketch_P is None:
                from .store import sketch_proj
                sketch_P = sketch_proj(kcg, cfg.sketch_dim)
        for si in range(n_k):
            c0 = kx["cg"][si] * kcg
            ps, nv = kx["pstart"][si], kx["nvalid"][si]
            if kscore_live:
                ks = query_aware_kscore_slot(Q_q[:, c0:c0 + kcg], kx["R"][si], A[:, ps:ps + nv],
                                             V_base[ps:ps + nv], cfg.head_dim)
                if np.isfinite(ks).all():
                    score_K[:, si] = ks * F32(sens)
                    continue
                if sketch_P is None:
                    from .store import sketch_proj
                    sketch_P = sketch_proj(kcg, cfg.sketch_dim)
                s_top = S.max(axis=1, keepdims=True)
                inv_margin = F32(1.0) / np.maximum(s_top - S, F32(EPS))
                vdiff = np.sqrt(((V_base[None] - O_base[:, None]) ** 2).sum(-1, dtype=F32), dtype=F32)
            pa = A[:, ps:ps + nv]
            mass = pa.sum(1, dtype=F32)
            boundary = (pa * inv_margin[:, ps:ps + nv]).sum(1, dtype=F32)
            pvd = (pa * vdiff[:, ps:ps + nv]).sum(1, dtype=F32)
            qs = Q_q[:, c0:c0 + kcg] @ sketch_P
            qdr = np.abs((qs * kx["sketch"][si][None]).sum(1, dtype=F32))
            score_K[:, si] = mass * qdr * boundary * pvd * F32(sens)
    score_V = None
    if want_v and (bv > 0 or route_mode):
        V_resid, v_starts, v_lens, v_err, _ = v_idx
        ar = np.arange(N)[None]
        v_mask = ((ar >= v_starts[:, None]) & (ar < (v_starts + v_lens)[:, None])).astype(F32)
        score_V = (A @ v_mask.T) * v_err[None]
        score_V = (score_V * F32(sens)).astype(F32)

    if route_mode:
        sK, sV = score_K, score_V  # route_selection normalises per kind itself
        if score_normalize and kind == "both":  # normalised copies for the diag
            if sK is not None:
                sK = sK / np.maximum(np.abs(sK).mean(1, keepdims=True, dtype=F32), F32(EPS))
            if sV is not None:
                sV = sV / np.maximum(np.abs(sV).mean(1, keepdims=True, dtype=F32), F32(EPS))
        score_K_raw, score_V_raw = score_K, score_V
    elif score_normalize and kind == "both" and score_K is not None and score_V is not None:
        nk = np.maximum(np.abs(score_K).mean(1, keepdims=True, dtype=F32), F32(EPS))
        nv_ = np.maximum(np.abs(score_V).mean(1, keepdims=True, dtype=F32), F32(EPS))
        sK, sV = score_K / nk, score_V / nv_
        if kscore_live:
            sK = sK * F32(lam_k)
            sV = sV * F32(lam_v)
    else:
        sK, sV = score_K, score_V

    sel_k = np.zeros((Qn, n_k), bool) if score_K is not None else None
    sel_v = np.zeros((Qn, n_v), bool) if score_V is not None else None
    if force_sel is not None:
        fk, fv = force_sel
        if sel_k is not None:
            sel_k[:] = fk
        if sel_v is not None:
            sel_v[:] = fv
    elif route_mode:
        for j in range(Qn):
            rk, rv = route_selection(None if score_K_raw is None else score_K_raw[j],
                                     None if score_V_raw is None else score_V_raw[j], bk, bv, policy,
                                     kind, score_normalize, A_row=A[j],
                                     adaptive_score=cfg.read_budget_mode == "adaptive_score",
                                     rel_thr=cfg.read_relative_threshold, abs_thr=cfg.read_absolute_threshold,
                                     min_keep=cfg.read_min_keep)
            if rk is not None:
                sel_k[j] = rk
            if rv is not None:
                sel_v[j] = rv
    elif policy == "joint" and kind == "both" and sK is not None and sV is not None:
        mb = (bk + bv) if (bk > 0 and bv > 0) else max(bk, bv)
        merged = np.concatenate([sK, sV], axis=1)
        mb = min(mb, merged.shape[1])
        top = topk_lowest_index(merged, mb)
        sm = np.zeros((Qn, n_k + n_v), bool)
        np.put_along_axis(sm, top, True, axis=1)
        sel_k, sel_v = sm[:, :n_k], sm[:, n_k:]
    else:
        if sK is not None and bk > 0:
            np.put_along_axis(sel_k, topk_lowest_index(sK, min(bk, n_k)), True, axis=1)
        if sV is not None and bv > 0:
            np.put_along_axis(sel_v, topk_lowest_index(sV, min(bv, n_v)), True, axis=1)
    if diag is not None:
        diag.update(score_K=score_K, score_V=score_V, score_K_r=sK, score_V_r=sV,
                    sel_k=sel_k, sel_v=sel_v)

    wK = None
    if sel_k is not None and sel_k.any():
        wK = np.zeros((Qn, N), F32)
        for si in range(n_k):
            c0 = kx["cg"][si] * kcg
            ps, nv = kx["pstart"][si], kx["nvalid"][si]
            qdr = Q_q[:, c0:c0 + kcg] @ kx["R"][si].T
            wK[:, ps:ps + nv] += sel_k[:, si].astype(F32)[:, None] * qdr
    V_resid_full = sel_tok = None
    if sel_v is not None and sel_v.any():
        V_resid, v_starts, v_lens, _, _ = v_idx
        ar = np.arange(N)[None]
        in_slot = (ar >= v_starts[:, None]) & (ar < (v_starts + v_lens)[:, None])
        covered = in_slot.any(0)
        t2s = in_slot.astype(np.int64).argmax(0)
        local = np.maximum(np.arange(N) - v_starts[t2s], 0)
        V_resid_full = np.zeros((N, D), F32)
        ci = np.nonzero(covered)[0]
        V_resid_full[ci] = V_resid[t2s[ci], local[ci]]
        sel_tok = sel_v[:, t2s] & covered[None]
    if k_mode == "exact" and wK is not None:
        delta = exact_softmax_correction(A, wK / F32(math.sqrt(D)), V_base, O_base, V_resid_full, sel_tok)
    else:
        if wK is not None:
            AwK = A * wK
            dK = AwK @ V_base - AwK.sum(1, keepdims=True, dtype=F32) * O_base
            delta = delta + F32(k_corr_scale) * dK
        if sel_tok is not None:
            delta = delta + (A * sel_tok.astype(F32)) @ V_resid_full
    return delta.astype(F32)


def base_attention(K_hat, V_hat, Qh):
    """attention.py:1015-1022 for a batch of query heads sharing one KV head."""
    K = np.asarray(K_hat, F32)
    V = np.asarray(V_hat, F32)
    Qf = np.asarray(Qh, F32)
    D = K.shape[1]
    S = (Qf @ K.T) * F32(1.0 / math.sqrt(D))
    A = softmax_rows(S)
    O = A @ V
    return S.astype(F32), A, O.astype(F32)


def decode_attention(cache: OCache, layer_id, Qh, page_ids_by_kvh=None, correction=True, diag=None, **corr_kw):
    """Decode attention for one sequence: Qh (Hq, D) fp16 -> (Hq, D) fp16.

    Per kv head: read_base_concat -> dequantize -> base attention ->
    batched joint correction over that kv head's query heads."""
    cfg = cache.cfg
    Hq, Hkv, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
    grp = Hq // Hkv
    out = np.zeros((Hq, D), F16)
    for h in range(Hkv):
        pids = cache.all_page_ids(layer_id, h) if page_ids_by_kvh is None else page_ids_by_kvh[h]
        heads = list(range(h * grp, (h + 1) * grp))
        if cfg.side_buffer:  # attention.py:997-1008: fp16 K_hat / V_hat, no dequantisation
            Kh, Vh, _ = cache.read_base_hat_concat(layer_id, h, pids)
            if Kh.shape[0] == 0:
                continue
            Kh, Vh = Kh.astype(F32), Vh.astype(F32)
        else:
            Kc, Ks, Vc, Vs, _ = cache.read_base_concat(layer_id, h, pids)
            if Kc.shape[0] == 0:
                continue
            Kh = Q.dequantize(Kc, Ks, cfg.group_size).astype(F32)
            Vh = Q.dequantize(Vc, Vs, cfg.group_size).astype(F32)
        Qg = np.asarray(Qh)[heads].astype(F32)
        S, A, O_base = base_attention(Kh, Vh, Qg)
        d = None if diag is None else diag.setdefault(h, {})
        O = O_base
        if correction:
            delta = vectorized_joint_correction(cache, layer_id, h, pids, Qg, S, A, Vh, O_base, diag=d, **corr_kw)
            O = O_base + delta
        if d is not None:
            d.update(S=S, A=A, O_base=O_base, V_hat=Vh, K_hat=Kh)
        out[heads] = O.astype(F16)
    return out


def prefill_stored(cache: OCache, layer_id, Qh, K_hat, V_hat, correction=True, diag=None, force_sel=None,
                   **corr_kw):
    """Prefill attention of ``CAREKVLayer.prefill`` in carekv_stored mode
    (layer.py:780-838) with the vectorized correction (layer.py:538-557).

    Qh (Hq, T, D) fp16 post-RoPE queries; K_hat / V_hat (Hkv, T, D) fp16 the
    page writer's dequantised prompt (write_pages_for_kv_head).  Per kv head:
    the causal base attention of _causal_attention_pure (fp32 scores with
    finfo(fp32).min above the diagonal, softmax weights cast to fp16,
    O_base = half(A @ V_hat)), then vectorized_joint_correction over the
    kv_group x T queries (head-major) against every page of the kv head,
    out = half(O_base + delta).  ``correction=False`` or no read budget gives
    the base (the any_read_budget short-circuit, layer.py:810-823).
    ``force_sel``: {kv head: (sel_k, sel_v)} replaces the selection of those
    kv heads (rows head-major, as the diag).  Returns (T, Hq, D) fp16."""
    cfg = cache.cfg
    Qh = np.asarray(Qh, F16)
    Hq, T, D = Qh.shape
    Hkv = cfg.num_kv_heads
    grp = Hq // Hkv
    mn = np.finfo(F32).min
    causal = np.where(np.arange(T)[None, :] > np.arange(T)[:, None], mn, F32(0)).astype(F32)
    any_budget = ((cfg.read_budget_mode in ("absolute", "adaptive_score") and (cfg.read_abs_k > 0 or cfg.read_abs_v > 0))
                  or cfg.read_budget_ratio > 0 or (cfg.read_budget_ratio_k or 0) > 0
                  or (cfg.read_budget_ratio_v or 0) > 0)
    out = np.zeros((Hq, T, D), F16)
    for h in range(Hkv):
        heads = list(range(h * grp, (h + 1) * grp))
        Kf = np.asarray(K_hat[h], F16).astype(F32)
        Vf = np.asarray(V_hat[h], F16).astype(F32)
        Qg = Qh[heads].astype(F32)
        S = (Qg @ Kf.T) / F32(math.sqrt(D)) + causal[None]
        m = S.max(axis=-1, keepdims=True)
        e = np.exp(S - m, dtype=F32)
        A = (e / e.sum(axis=-1, keepdims=True, dtype=F32)).astype(F16)
        O_base = (A.astype(F32) @ Vf).astype(F16)
        if not (correction and any_budget):
            out[heads] = O_base
            continue
        pids = cache.all_page_ids(layer_id, h)
        d = None if diag is None else diag.setdefault(h, {})
        delta = vectorized_joint_correction(cache, layer_id, h, pids, Qg.reshape(-1, D), S.reshape(-1, T),
                                            A.astype(F32).reshape(-1, T), Vf, O_base.astype(F32).reshape(-1, D),
                                            diag=d, force_sel=None if force_sel is None else force_sel.get(h),
                                            **corr_kw)
        out[heads] = (O_base.astype(F32) + delta.reshape(grp, T, D)).astype(F16)
        if d is not None:
            d.update(S=S.reshape(-1, T), A=A.astype(F32).reshape(-1, T), V_hat=Vf, K_hat=Kf)
    return out.transpose(1, 0, 2)


def causal_attention_pure(Qh, K, V, causal=True, rows=None):
    """layer.py:935-972: scores = fp32(Q) . fp32(K) / sqrt(D); causal mask with
    finfo(fp32).min above the diagonal; softmax in fp32; weights cast to
    fp16; O = weights @ V with fp32 accumulation, returned in fp16.

    Qh (Hq, T, D) fp16, K/V (Hkv, T, D) fp16; query head h reads kv head
    h // (Hq / Hkv) (repeat_interleave, layer.py:774-775).  ``rows``
    restricts the computation to those query rows (for long sequences).
    Returns (O (Hq, n_rows, D) fp16, lse (Hq, n_rows) fp32)."""
    Qh = np.asarray(Qh, dtype=F16)
    K = np.asarray(K, dtype=F16)
    V = np.asarray(V, dtype=F16)
    Hq, T, D = Qh.shape
    grp = Hq // K.shape[0]
    rows = np.arange(T) if rows is None else np.asarray(rows)
    out = np.zeros((Hq, len(rows), D), dtype=F16)
    lse = np.zeros((Hq, len(rows)), dtype=F32)
    inv = F32(math.sqrt(D))
    mn = np.finfo(F32).min
    for h in range(Hq):
        Kf = K[h // grp].astype(F32)
        Vf = V[h // grp].astype(F32)
        S = (Qh[h, rows].astype(F32) @ Kf.T) / inv  # (n_rows, T)
        if causal:
            S = S + np.where(np.arange(T)[None, :] > rows[:, None], mn, F32(0)).astype(F32)
        m = S.max(axis=-1, keepdims=True)
        e = np.exp(S - m, dtype=F32)
        z = e.sum(axis=-1, keepdims=True, dtype=F32)
        A = (e / z).astype(F16)
        out[h] = (A.astype(F32) @ Vf).astype(F16)
        lse[h] = (m[:, 0] + np.log(z[:, 0])).astype(F32)
    return out, lse


def prefill_eval(Qh, K, V, K_hat, V_hat, *, ratio, min_residuals=1, kind="both", v_score="output_aware",
                 normalize=False, k_corr_scale=0.1, diag=None, force_sel=None, o_base=None, rows=None):
    """``CAREKVLayer`` prefill in ``carekv_eval`` mode (layer.py:792-806): the
    causal base attention over K_hat / V_hat (``causal_attention_pure``,
    fp16 weights A and fp16 O_base), then
    ``_apply_sparse_prefill_correction_eval`` (layer.py:363-456) per (query
    head, row t) with the full in-memory residuals r_k = half(K - K_hat),
    r_v = half(V - V_hat) (layer.py:770-775):
      n = t + 1, k = min(max(min_residuals, int(n * ratio)), n)
      v_diff_t = ||V_hat_t - o||, qdot_t = (r_k,t . q) / sqrt(D)
      v_score = a ||r_v|| v_diff (output_aware) or a ||r_v|| (norm)
      k_score = a |qdot| v_diff
      score = v, k, v + k or v / mean|v| + k / mean|k| (clamped 1e-8)
      top-k tokens (ties to the lower index);
      dO_V = sum a r_v, dO_K = sum a clamp(qdot, -2, 2) (V_hat - o)
      out = half(o + dO_V + k_corr_scale dO_K)  (terms of the kind only).
    Qh (Hq, T, D) fp16 post-RoPE; K, V, K_hat, V_hat (Hkv, T, D) fp16.
    ``diag`` receives {(h, t): (selected token indices, scores)};
    ``force_sel`` maps (h, t) to the token indices to use instead of the
    top-k; ``o_base`` (Hq, T, D) fp16 replaces the base output O (the
    weights A stay the fp32 softmax cast to fp16), to hold the correction
    alone to a device whose base attention rounds differently.
    ``rows`` (needs ``o_base``): only those rows t are corrected (each row's
    scores and weights computed from that row alone; the other rows keep
    O), for long prompts.
    Returns (T, Hq, D) fp16."""
    Qh = np.asarray(Qh, F16)
    Hq, T, D = Qh.shape
    Hkv = np.asarray(K).shape[0]
    grp = Hq // Hkv
    assert rows is None or o_base is not None, "rows needs o_base"
    O = causal_attention_pure(Qh, K_hat, V_hat)[0] if o_base is None else np.asarray(o_base, F16)
    rk = (np.asarray(K, F16).astype(F32) - np.asarray(K_hat, F16).astype(F32)).astype(F16).astype(F32)
    rv = (np.asarray(V, F16).astype(F32) - np.asarray(V_hat, F16).astype(F32)).astype(F16).astype(F32)
    Vh = np.asarray(V_hat, F16).astype(F32)
    Kh = np.asarray(K_hat, F16).astype(F32)
    scale = F32(1.0 / math.sqrt(D))
    out = O.astype(F32).copy()
    mn = np.finfo(F32).min
    row_list = list(range(T)) if rows is None else sorted(int(t) for t in rows)

    def weights(q, hk, ts):
        # layer.py:955-964 on rows ts: fp32 scores / sqrt(D), causal mask,
        # softmax, cast to fp16
        S = (q[ts] @ Kh[hk].T) / F32(math.sqrt(D))
        S = S + np.where(np.arange(T)[None, :] > np.asarray(ts)[:, None], mn, F32(0)).astype(F32)
        m = S.max(axis=-1, keepdims=True)
        e = np.exp(S - m, dtype=F32)
        return (e / e.sum(axis=-1, keepdims=True, dtype=F32)).astype(F16).astype(F32)

    for h in range(Hq):
        hk = h // grp
        q = Qh[h].astype(F32)
        rvn = np.sqrt((rv[hk] * rv[hk]).sum(-1, dtype=F32))      # (T,)
        if rows is None:
            A = weights(q, hk, np.arange(T))
            qdot_all = (q @ rk[hk].T) * scale                    # (T rows, T tokens)
        for t in row_list:
            n = t + 1
            k = min(max(int(min_residuals), int(n * ratio)), n)
            if k <= 0:
                continue
            if rows is None:
                a, qd = A[t, :n], qdot_all[t, :n]
            else:
                a = weights(q, hk, [t])[0, :n]
                qd = ((q[t:t + 1] @ rk[hk].T) * scale)[0, :n]
            o = O[h, t].astype(F32)
            vdiff = np.sqrt(((Vh[hk, :n] - o[None, :]) ** 2).sum(-1, dtype=F32))
            vs = a * rvn[:n] if v_score == "norm" else a * rvn[:n] * vdiff
            ks = a * np.abs(qd) * vdiff
            if kind == "v":
                sc = vs
            elif kind == "k":
                sc = ks
            elif normalize:
                vm = max(float(np.abs(vs).mean(dtype=F32)), 1e-8)
                km = max(float(np.abs(ks).mean(dtype=F32)), 1e-8)
                sc = vs / F32(vm) + ks / F32(km)
            else:
                sc = vs + ks
            if force_sel is not None and (h, t) in force_sel:
                idx = force_sel[(h, t)]
            else:
                idx = np.argsort(-sc, kind="stable")[:k]  # ties to the lower index
            idx = np.sort(np.asarray(idx, dtype=np.int64))
            if diag is not None:
                diag[(h, t)] = (idx, sc)
            a_s = a[idx]
            dv = (a_s[:, None] * rv[hk, idx]).sum(0, dtype=F32) if kind in ("v", "both") else np.zeros(D, F32)
            if kind in ("k", "both"):
                qc = np.clip(qd[idx], -2.0, 2.0)
                dk = ((a_s * qc)[:, None] * (Vh[hk, idx] - o[None, :])).sum(0, dtype=F32)
            else:
                dk = np.zeros(D, F32)
            out[h, t] = o + dv + F32(k_corr_scale) * dk
    return out.astype(F16).transpose(1, 0, 2)
