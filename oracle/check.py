"""Selection and output comparison helpers for the parity checks.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): used by ``tests/``
and by ``bench.py``'s ``cpu_baseline`` leg to compare the HIP path's output
and selected candidates with the oracle's.

Candidate ids are (kind, page, sub): kind 0 = K slot of channel group
``sub``, kind 1 = V block ``sub``, in the reference's candidate order
(``attention.py:386-441,540-573``: page-major, stored slots only).
"""
from __future__ import annotations

import numpy as np

F16, F32 = np.float16, np.float32


def oracle_candidates(oc, layer, h, n_pages):
    """Candidate ids (kind, page, sub) of one kv head in the reference's index
    order: K slots of pages with metadata, V blocks that start inside the
    page's valid rows (``attention.py:409-421,548-570``)."""
    cfg = oc.cfg
    K, V = [], []
    for p in range(n_pages):
        m = oc.meta_table[layer][h][p]
        nv = int(oc.valid_tokens[layer, h, p])
        if nv == 0 or m is None:
            continue
        for cg, s in enumerate(m.k_residual_slots):
            if s >= 0:
                K.append((0, p, cg))
        for vb, s in enumerate(m.v_residual_slots):
            if s >= 0 and vb * cfg.v_token_block < nv:
                V.append((1, p, vb))
    return K, V


def decode_diag(code_row):
    """The HIP diag row (kind<<30 | page<<3 | sub, -1 padded) as id tuples."""
    out = []
    for x in code_row:
        x = int(x)
        if x < 0:
            break
        out.append((x >> 30, (x >> 3) & ((1 << 27) - 1), x & 7))
    return out


def oracle_selection(diag_h, Kc, Vc):
    """Per query row: the set of candidate ids the oracle selected."""
    rows = []
    sk, sv = diag_h["sel_k"], diag_h["sel_v"]
    for j in range(sk.shape[0] if sk is not None else sv.shape[0]):
        s = set()
        if sk is not None:
            s |= {Kc[i] for i in np.nonzero(sk[j])[0]}
        if sv is not None:
            s |= {Vc[i] for i in np.nonzero(sv[j])[0]}
        rows.append(s)
    return rows


def ties_explain(mine: set, ref: set, diag_h, Kc, Vc, j, eps=1e-4):
    """True if every disagreement is between candidates whose normalised
    scores sit within eps (relative) of the selection boundary (the oracle's
    k-th selected score)."""
    if mine == ref:
        return True
    sK, sV = diag_h["score_K_r"], diag_h["score_V_r"]
    vals = {}
    if sK is not None:
        vals.update({c: float(sK[j, i]) for i, c in enumerate(Kc)})
    if sV is not None:
        vals.update({c: float(sV[j, i]) for i, c in enumerate(Vc)})
    ref_vals = sorted((vals[c] for c in ref), reverse=True)
    kth = ref_vals[-1] if ref_vals else 0.0
    for c in mine ^ ref:
        if c not in vals or abs(vals[c] - kth) > eps * max(abs(kth), 1e-30):
            return False
    return True


def compare_selection(diag_rows, odiag_h, Kc, Vc, eps=1e-4, per_kind=False):
    """Compare the HIP diag rows of a kv head's query heads with the oracle's
    selection.  Returns (exact, tie, bad): rows equal, rows that differ only
    across an epsilon tie, rows that differ otherwise.  ``per_kind`` checks
    the K and the V selections separately (separate / route policies)."""
    ref_rows = oracle_selection(odiag_h, Kc, Vc)
    exact = tie = bad = 0
    for j, ref in enumerate(ref_rows):
        mine = set(decode_diag(diag_rows[j]))
        if mine == ref:
            exact += 1
            continue
        if per_kind:
            ok = all(ties_explain({c for c in mine if c[0] == k}, {c for c in ref if c[0] == k}, odiag_h, Kc, Vc,
                                  j, eps) for k in (0, 1))
        else:
            ok = ties_explain(mine, ref, odiag_h, Kc, Vc, j, eps)
        if ok:
            tie += 1
        else:
            bad += 1
    return exact, tie, bad


def output_errors(out, ref, atol=2e-3):
    """(max-abs error, relative L2 error, worst ratio of the error to the bar
    max(atol, one fp16 ulp of ref)) of an fp16 output against the oracle's;
    the output passes the bar where the last value is <= 1."""
    o = np.asarray(out, F32)
    r = np.asarray(ref, F32)
    if o.size == 0:
        return 0.0, 0.0, 0.0
    err = np.abs(o - r)
    rel = float(np.linalg.norm(o - r) / max(np.linalg.norm(r), 1e-30))
    ulp = np.spacing(np.abs(np.asarray(ref).astype(F16))).astype(F32)
    return float(err.max()), rel, float((err / np.maximum(F32(atol), ulp)).max())


def oracle_slice_from_device(cache, seq, kvh, layer=0, **cfg_kw):
    """An oracle cache holding one (sequence, kv head) of a device cache (a
    ``care_kv.CAREKVCache``, read through its public tensors), as a one-layer,
    one-kv-head ``OCache`` whose pages, metadata and slot arena are copies of
    the device's.  ``cfg_kw`` sets the oracle config's read knobs (query
    heads of the group, budgets, policy); the cache geometry comes from the
    device cache."""
    from .cache import OCache, OCfg, OMeta
    dc = cache.cfg
    P = cache.num_pages(layer, kvh, seq)
    kw = dict(num_layers=1, num_kv_heads=1, head_dim=dc.head_dim, page_size=dc.page_size, max_pages=max(P, 1),
              base_bits=dc.base_bits, group_size=dc.group_size, k_channel_group=dc.k_channel_group,
              v_token_block=dc.v_token_block, sketch_dim=dc.sketch_dim, base_quantizer=dc.base_quantizer,
              scale_quant=dc.scale_quant, residual_bits=dc.residual_bits,
              layer_sensitivity=[float(dc.layer_sensitivity[layer])])
    kw.update(cfg_kw)
    oc = OCache(OCfg(**kw), max_slots=cache.n_slots)
    g = lambda t: t[layer, kvh, seq, :P].cpu().numpy()  # noqa: E731
    if oc.cfg.side_buffer and getattr(cache, "kivi_packed", False):
        # the packed KIVI base, read back as the side buffer it stands for
        kh, vh, lens = cache.read_base_hat_concat(layer, kvh, list(range(P)), seq=seq)
        kh, vh, r = kh.cpu().numpy(), vh.cpu().numpy(), 0
        for p, n in enumerate(lens):
            oc.base_K_hat_fp16[0, 0, p, :n] = kh[r:r + n]
            oc.base_V_hat_fp16[0, 0, p, :n] = vh[r:r + n]
            r += n
    elif oc.cfg.side_buffer:  # fp16 rows of the side buffer
        oc.base_K_hat_fp16[0, 0, :P] = g(cache.kcodes).view(F16)
        oc.base_V_hat_fp16[0, 0, :P] = g(cache.vcodes).view(F16)
    else:
        oc.base_K_codes[0, 0, :P] = g(cache.kcodes)
        oc.base_V_codes[0, 0, :P] = g(cache.vcodes)
        oc.base_K_scale[0, 0, :P] = g(cache.kscale)
        oc.base_V_scale[0, 0, :P] = g(cache.vscale)
        if oc.base_K_scale_master is not None:
            oc.base_K_scale_master[0, 0, :P] = g(cache.kmaster)
            oc.base_V_scale_master[0, 0, :P] = g(cache.vmaster)
    oc.valid_tokens[0, 0, :P] = g(cache.valid)
    oc.k_residual_buf[:] = cache.k_res[seq].cpu().numpy()
    oc.v_residual_buf[:] = cache.v_res[seq].cpu().numpy()
    oc.k_residual_scale[:, 0] = cache.k_res_scale[seq].cpu().numpy()
    oc.v_residual_scale[:, 0] = cache.v_res_scale[seq].cpu().numpy()
    hm, ks, vs, ke, ve, sk = (g(cache.has_meta), g(cache.k_slot), g(cache.v_slot), g(cache.k_err),
                              g(cache.v_err), g(cache.k_sketch))
    for p in range(P):
        if hm[p]:
            oc.meta_table[0][0][p] = OMeta(page_id=p, layer_id=0, kv_head=0, token_start=p * dc.page_size,
                                           num_tokens=int(oc.valid_tokens[0, 0, p]),
                                           k_residual_slots=ks[p].tolist(), v_residual_slots=vs[p].tolist(),
                                           k_error_norm=ke[p], v_error_norm=ve[p], k_sketch=sk[p])
    oc.next_page[0][0] = P
    return oc


def forced_selection(diag_rows, Kc, Vc):
    """(sel_k, sel_v) boolean masks of the HIP diag rows over the oracle's
    candidate lists, for recomputing the oracle's output under the HIP
    path's selection (``vectorized_joint_correction(force_sel=...)``)."""
    ki = {c: i for i, c in enumerate(Kc)}
    vi = {c: i for i, c in enumerate(Vc)}
    fk = np.zeros((len(diag_rows), len(Kc)), bool)
    fv = np.zeros((len(diag_rows), len(Vc)), bool)
    for j, row in enumerate(diag_rows):
        for c in decode_diag(row):
            if c[0] == 0:
                fk[j, ki[c]] = True
            else:
                fv[j, vi[c]] = True
    return fk, fv
