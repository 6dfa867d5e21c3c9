"""Decode attention with CARE-KV residual correction (host side).

``decode_attention`` launches the fused HIP kernel for a batch of
sequences of one layer.  It computes, per (sequence, kv head), what the
reference computes with ``read_base_concat`` + ``dequantize`` + base
attention (attention.py:996-1022) followed by ``vectorized_joint_correction``
over the kv head's query heads (attention.py:576-957): the comb+ex selector
(CAREKV_KSCORE_LIVE=1) or the sketch-proxy K score (CAREKV_KSCORE_LIVE=0,
attention.py:718-725), per-query score normalisation, joint or separate
top-k, and the exact (or linear) K correction.  ``CAREKVAttention`` and
``CAREKVMultiHeadAttention`` keep the reference's per-head / multi-head entry
points (attention.py:964-1077) on top of it.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from .cache import CAREKVCache, get_sketch_proj, to_device
from .config import CacheConfig, ReadKnobs, any_read_budget, resolve_read_knobs

KIND_CODE = {"both": 0, "k": 1, "v": 2}

# ------------------------------------------------------------------ debug stats
# Process-global read counters (layer.py:90-126): with CAREKV_DEBUG_STATS=1
# every decode / prefill-correction launch adds, on the device, the K slots
# and V blocks it selected and the queries it corrected (the select kernel's
# atomics); get_debug_stats reads them back.
_READ_COUNTS: dict = {}


def debug_stats_enabled() -> bool:
    """layer.py:116-117."""
    return os.environ.get("CAREKV_DEBUG_STATS", "0") == "1"


def _read_counts_ptr(device) -> int:
    if not debug_stats_enabled():
        return 0
    key = str(device)
    t = _READ_COUNTS.get(key)
    if t is None:
        t = torch.zeros(3, dtype=torch.int64, device=device)
        _READ_COUNTS[key] = t
    return t.data_ptr()


# Host-side sums of the reference's debug dict: the delta norms of the
# per-query correction (apply_slot_corrections / CAREKVAttention with a
# debug dict, attention.py:358-372) and the token-importance dispersion of
# the carekv_stored prefill (CAREKV_DUMP_IMPORTANCE=1, layer.py:477-502).
# The batched decode and prefill kernels, like the reference's vectorized
# path (attention.py:945-947), count slot reads only.
_HOST_STATS = {"delta_v_norm_sum": 0.0, "delta_k_norm_sum": 0.0, "delta_o_norm_sum": 0.0, "o_base_norm_sum": 0.0,
               "imp_gini_sum": 0.0, "imp_norm_entropy_sum": 0.0, "imp_top1pct_mass_sum": 0.0, "imp_count": 0}
# layer id -> [gini sum, normalised entropy sum, top-1% mass sum, count]
_IMP_PER_LAYER: dict = {}


def get_debug_stats() -> dict:
    """layer.py:120-121: a snapshot of the debug counters.  k_slots_read /
    v_slots_read / n_queries are counted on the device by every corrected
    launch (read back here); the delta-norm sums accumulate on the per-query
    path and the importance sums in the carekv_stored prefill."""
    k = v = n = 0
    for t in _READ_COUNTS.values():
        a, b, c = (int(x) for x in t.tolist())
        k, v, n = k + a, v + b, n + c
    return {"v_slots_read": v, "k_slots_read": k, "n_queries": n, **_HOST_STATS}


def reset_debug_stats() -> None:
    """layer.py:123-126."""
    for t in _READ_COUNTS.values():
        t.zero_()
    for key in _HOST_STATS:
        _HOST_STATS[key] = 0 if key == "imp_count" else 0.0
    _IMP_PER_LAYER.clear()


def get_imp_per_layer() -> dict:
    """layer.py:107-114: per-layer means of the token-importance dispersion
    (empty unless CAREKV_DUMP_IMPORTANCE=1 and CAREKV_DEBUG_STATS=1 were set
    during a carekv_stored prefill)."""
    return {lid: dict(gini=g / c, norm_entropy=e / c, top1pct_mass=t / c, count=c)
            for lid, (g, e, t, c) in _IMP_PER_LAYER.items() if c}


def importance_probe(layer_id: int, q: torch.Tensor, k_hat: torch.Tensor) -> None:
    """layer.py:477-502 for one prompt: the attention mass each key gets
    from every query head and causal prompt row of the base attention over
    K_hat (fp32 softmax), its Gini coefficient, entropy normalised by
    log(N) and the mass share of the top 1% of keys, added to the debug
    sums and the layer's.  q (Hq, T, D), k_hat (Hkv, T, D)."""
    Hq, T, D = q.shape
    grp = Hq // k_hat.shape[0]
    mass = torch.zeros(T, dtype=torch.float32, device=q.device)
    causal = torch.ones(T, T, dtype=torch.bool, device=q.device).tril_()
    for h in range(Hq):
        s = (q[h].float() @ k_hat[h // grp].float().transpose(0, 1)) / math.sqrt(D)
        mass += torch.softmax(s.masked_fill(~causal, float("-inf")), dim=-1).sum(0)
    tot = mass.sum().clamp_min(1e-9)
    p = mass / tot
    ent = float(-(p * (p + 1e-12).log()).sum() / math.log(max(T, 2)))
    srt = torch.sort(mass).values
    i = torch.arange(1, T + 1, device=q.device, dtype=srt.dtype)
    gini = float(((2 * i - T - 1) * srt).sum() / (T * srt.sum().clamp_min(1e-9)))
    top1 = float(torch.topk(mass, max(1, T // 100)).values.sum() / tot)
    _HOST_STATS["imp_gini_sum"] += gini
    _HOST_STATS["imp_norm_entropy_sum"] += ent
    _HOST_STATS["imp_top1pct_mass_sum"] += top1
    _HOST_STATS["imp_count"] += 1
    acc = _IMP_PER_LAYER.setdefault(layer_id, [0.0, 0.0, 0.0, 0])
    acc[0] += gini
    acc[1] += ent
    acc[2] += top1
    acc[3] += 1


def decode_read_mode(cfg: CacheConfig, layer: int):
    """(correction on, read knobs) of a decode step through
    ``CAREKVLayer.decode_step`` / ``CAREKVMultiHeadAttention``.

    ``cfg.compat``: as the reference's decode path, which corrects only when
    read_budget_ratio > 0 (attention.py:1025) and then selects per query
    head through ResidualRouter.route (apply_slot_corrections,
    attention.py:208-374; the router reads no CAREKV_KSCORE_LIVE), i.e. with
    the sketch-proxy K score.  Otherwise the correction runs whenever a read
    budget is set (layer.py:813-819's test) with the knobs of
    ``resolve_read_knobs`` (the query-aware score under CAREKV_KSCORE_LIVE=1)."""
    knobs = resolve_read_knobs(cfg, layer)
    if cfg.compat:
        knobs.kscore_live = False
        return cfg.read_budget_ratio > 0, knobs
    return any_read_budget(cfg), knobs


def default_split_pages(max_pages: int, rows: int) -> int:
    """Pages per work-group of the streaming pass, a multiple of 16 (4 waves
    x 4-page windows): long enough that each wave's start-up (q staging, the
    first window's loads, the split merge) spreads over several windows --
    half a row, at most 256 pages -- and short enough that the grid keeps at
    least CAREKV_DECODE_MIN_WGS (default 1024: four per CU) work-groups."""
    min_wgs = max(1, int(os.environ.get("CAREKV_DECODE_MIN_WGS", "1024")))
    P, R = max(1, max_pages), max(1, rows)
    sp = max(16, min(256, -(-P // 2), (P * R) // min_wgs))
    return (sp + 15) // 16 * 16


def _read_params(cache: CAREKVCache, layer: int, knobs: ReadKnobs, *, batch: int, n_heads: int, correction: bool,
                 split_pages: int, max_pages: int, seq_ptr: int = 0, np_ptr: int = 0):
    """carekv_decode_params of the resolved read knobs (the sketch proxy's
    projection is set by the caller)."""
    cfg = cache.cfg
    return _lib.DecodeParams(
        batch=batch, n_heads=n_heads, seq_slot=seq_ptr, n_pages=np_ptr, max_pages_used=max_pages,
        sm_scale=float(np.float32(1.0 / math.sqrt(cfg.head_dim))), sensitivity=float(cfg.layer_sensitivity[layer]),
        correction=int(bool(correction)), kind=KIND_CODE[knobs.kind], joint=int(knobs.joint),
        normalize=int(knobs.normalize), k_exact=int(knobs.k_exact), k_corr_scale=knobs.k_corr_scale,
        lambda_k=knobs.lambda_k, lambda_v=knobs.lambda_v, budget_ratio=int(knobs.budget_ratio),
        abs_k=knobs.abs_k, abs_v=knobs.abs_v, ratio_k=knobs.ratio_k, ratio_v=knobs.ratio_v,
        k_cap=cache.k_cap, v_cap=cache.v_cap, split_pages=int(split_pages),
        route_policy=int(knobs.route_policy), adaptive_score=int(bool(knobs.adaptive_score)),
        rel_threshold=float(knobs.rel_threshold), abs_threshold=float(knobs.abs_threshold),
        min_keep=int(knobs.min_keep))


def prefill_correction(cache: CAREKVCache, layer: int, q: torch.Tensor, k_hat: torch.Tensor, v_hat: torch.Tensor,
                       lse: torch.Tensor, seq: int = 0, *, knobs: Optional[ReadKnobs] = None,
                       split_pages: Optional[int] = None, diag_cap: int = 0, rows_per_call: Optional[int] = None):
    """The prefill-time correction of ``carekv_stored`` mode (layer.py:780-838)
    over all kv_group x T queries, for the prompt that sequence ``seq`` of
    the cache holds (written by ``write_prefill`` from token 0).  With
    ``knobs.kscore_live`` it is the vectorized correction of
    correction_impl=vectorized (layer.py:538-557); without, the per-(head,
    row) apply_slot_corrections over ResidualRouter.route of
    correction_impl=cached / python (layer.py:573-640, the router's sketch
    proxy score, its policies and thresholds), which the reference's own test
    holds equal to the vectorized form over the same scores
    (tests/test_vectorized_carekv.py:83-162).

    q (T, Hq, D) fp16 post-RoPE queries; k_hat / v_hat (Hkv, T, D) fp16 the
    page writer's dequantised prompt (``quant_dequant`` for the uniform
    base, the KIVI quant-dequant for the side-buffer bases); lse (Hq, T)
    fp32 from ``prefill_attention(..., return_lse=True)`` over the same
    K_hat / V_hat.  Returns the corrected attention output (T, Hq, D) fp16,
    and with ``diag_cap > 0`` the selected candidates per (row, head)."""
    cfg: CacheConfig = cache.cfg
    if knobs is None:
        knobs = resolve_read_knobs(cfg, layer)
    T, Hq, D = q.shape
    Hkv = cfg.num_kv_heads
    if (Hq, D) != (cfg.num_heads, cfg.head_dim) or k_hat.shape != (Hkv, T, D) or v_hat.shape != (Hkv, T, D) \
            or lse.shape != (Hq, T):
        raise ValueError("prefill_correction: q (T, Hq, D), k_hat / v_hat (Hkv, T, D), lse (Hq, T) expected")
    dev = cache.device
    q = q.to(torch.float16).contiguous()
    k_hat = k_hat.to(torch.float16).contiguous()
    v_hat = v_hat.to(torch.float16).contiguous()
    lse = lse.to(torch.float32).contiguous()
    pages = -(-T // cfg.page_size)
    if cache.num_pages(layer, 0, seq) != pages:
        raise ValueError(f"sequence {seq} holds {cache.num_pages(layer, 0, seq)} pages, the prompt needs {pages}: "
                         "the cache must hold exactly the prompt")
    if rows_per_call is None:  # bound the workspace: rows x pages x query heads <= 2^23 (about 0.6 GB)
        rows_per_call = max(1, min(T, (1 << 23) // max(1, pages * Hq)))
    if split_pages is None:
        split_pages = default_split_pages(pages, rows_per_call * Hkv)
    lib = _lib.load()
    a = cache.arena(layer)
    out = torch.empty(T, Hq, D, dtype=torch.float16, device=dev)
    diag = torch.empty(T, Hq, diag_cap, dtype=torch.int32, device=dev) if diag_cap > 0 else None
    dp = _read_params(cache, layer, knobs, batch=0, n_heads=Hq, correction=True, split_pages=split_pages,
                      max_pages=pages)
    if not knobs.kscore_live:  # the router's sketch-proxy K score
        dp.k_proxy = 1
        dp.sketch_proj = get_sketch_proj(cfg.head_dim, cfg.k_channel_group, cfg.sketch_dim, dev).data_ptr()
    dp.read_counts = _read_counts_ptr(dev)
    for r0 in range(0, T, rows_per_call):
        n = min(rows_per_call, T - r0)
        pp = _lib.PrefillCorrParams(seq=seq, n_tokens=T, row_begin=r0, n_rows=n, k_hat=k_hat.data_ptr(),
                                    v_hat=v_hat.data_ptr(), lse=lse.data_ptr())
        nbytes = int(lib.carekv_prefill_correct_workspace_bytes(a, dp, pp))
        if nbytes < 0:
            raise _lib.CarekvError(f"carekv_prefill_correct_workspace_bytes rejected the parameters: "
                                   f"{lib.carekv_last_error().decode()}")
        ws = cache.workspace("prefill_correct", nbytes)
        _lib.check(lib.carekv_prefill_correct(a, dp, pp, q[r0].data_ptr(), out[r0].data_ptr(), ws.data_ptr(),
                                              ws.numel(), None if diag is None else diag[r0].data_ptr(),
                                              int(diag_cap), _lib.stream_ptr(dev)), "carekv_prefill_correct")
        if _lib.check_enabled():
            _lib.check_status(ws, 0, "carekv_prefill_correct")
    return (out, diag) if diag_cap > 0 else out


def decode_attention(cache: CAREKVCache, layer: int, q: torch.Tensor, seqs: Optional[Sequence[int]] = None, *,
                     correction: bool = True, knobs: Optional[ReadKnobs] = None, split_pages: Optional[int] = None,
                     diag_cap: int = 0, out: Optional[torch.Tensor] = None, phase_events=None,
                     no_alloc: bool = False, n_pages: Optional[Sequence[int]] = None, count_reads: bool = True):
    """q: (B, Hq, D) fp16 post-RoPE queries of B sequences -> (B, Hq, D) fp16.

    With ``diag_cap > 0`` also returns the selected candidates per query
    head as an int32 (B, Hq, diag_cap) tensor (kind<<30 | page<<3 | sub, -1
    padded), for parity checks.  ``phase_events``: optional sequence of 5
    recorded torch.cuda.Event (timing enabled), re-recorded on the launch
    stream around the streaming, select, apply and combine kernels.

    ``no_alloc``: run through ``carekv_decode_attn_static``, whose workspace
    is the library's per-GPU static array (at most
    ``_lib.STATIC_SCRATCH_BYTES``) instead of a buffer the cache owns; the
    library call then allocates nothing (pass ``out``).  ``n_pages``: per
    sequence, attend to its first n pages only (default: all of them).
    ``count_reads=False`` keeps the launch out of the debug read counters."""
    cfg: CacheConfig = cache.cfg
    if q.dim() == 2:
        q = q.unsqueeze(0)
    B, Hq, D = q.shape
    assert D == cfg.head_dim and Hq == cfg.num_heads
    seqs = list(range(B)) if seqs is None else list(seqs)
    if knobs is None:
        knobs = resolve_read_knobs(cfg, layer)
    q = q.to(torch.float16).contiguous()
    npages = cache.next_page[layer, 0, np.asarray(seqs, dtype=np.int64)].astype(np.int32)
    if n_pages is not None:
        npages = np.minimum(npages, np.asarray(list(n_pages), dtype=np.int32))
    max_np = int(npages.max()) if B else 0
    dev = cache.device
    key = (tuple(seqs), npages.tobytes())
    meta = cache._row_tables.get(key)
    if meta is None:  # device row table, reused while the batch is unchanged
        meta = to_device(np.stack([np.array(seqs, dtype=np.int32), npages]), dev)
        if len(cache._row_tables) > 64:
            cache._row_tables.clear()
        cache._row_tables[key] = meta
    if split_pages is None:
        split_pages = default_split_pages(max_np, B * cfg.num_kv_heads)
    dp = _read_params(cache, layer, knobs, batch=B, n_heads=Hq, correction=correction, split_pages=split_pages,
                      max_pages=max_np, seq_ptr=meta[0].data_ptr(), np_ptr=meta[1].data_ptr())
    if cache.kivi_packed and B:  # the packed prefix and the fp16 tail run as separate page ranges
        pp = np.minimum(npages, cache.n_packed[seqs])
        dp.packed_pages_used, dp.tail_pages_used = int(pp.max()), int((npages - pp).max())
    if correction and not knobs.kscore_live:
        P = get_sketch_proj(cfg.head_dim, cfg.k_channel_group, cfg.sketch_dim, dev)
        dp.k_proxy = 1
        dp.sketch_proj = P.data_ptr()
    if correction and count_reads:
        dp.read_counts = _read_counts_ptr(dev)
    ev_arr = None
    if phase_events is not None:
        if len(phase_events) != 5:
            raise ValueError("phase_events needs 5 events")
        ev_arr = (ctypes.c_void_p * 5)(*[int(e.cuda_event) for e in phase_events])
        dp.phase_events = ctypes.cast(ev_arr, ctypes.c_void_p)
    lib = _lib.load()
    a = cache.arena(layer)
    if out is None:
        out = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)
    diag = torch.empty(B, Hq, diag_cap, dtype=torch.int32, device=dev) if diag_cap > 0 else None
    if no_alloc:
        _lib.check(lib.carekv_decode_attn_static(a, dp, q.data_ptr(), out.data_ptr(),
                                                 None if diag is None else diag.data_ptr(), int(diag_cap),
                                                 _lib.stream_ptr(dev)), "carekv_decode_attn_static")
        return (out, diag) if diag_cap > 0 else out
    nbytes = int(lib.carekv_decode_workspace_bytes(a, dp))
    if nbytes < 0:
        raise _lib.CarekvError("carekv_decode_workspace_bytes rejected the parameters")
    ws = cache.workspace("decode", nbytes)
    _lib.check(lib.carekv_decode_attn(a, dp, q.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                      None if diag is None else diag.data_ptr(), int(diag_cap),
                                      _lib.stream_ptr(dev)), "carekv_decode_attn")
    if _lib.check_enabled():
        _lib.check_status(ws, 0, "carekv_decode_attn")
    return (out, diag) if diag_cap > 0 else out


def apply_slot_corrections(cache: CAREKVCache, cfg: CacheConfig, router, layer_id: int, kv_head: int, page_ids,
                           q: torch.Tensor, s_base=None, a_base=None, V_base=None, O_base=None, kind: str = "both",
                           k_corr_scale: float = 1.0, score_normalize: bool = False, debug_stats=None,
                           slot_cache=None, seq: int = 0) -> torch.Tensor:
    """attention.py:208-374: the correction dO (D,) for one query from the
    stored slots the router selects (ResidualRouter.route's score, linear or
    exact K correction per CAREKV_K_CORRECTION_MODE), as the decode kernels
    compute it from the cache pages.  dO is returned as the fp32 difference
    between the corrected fp16 output and O_base (the reference's callers
    form half(O_base + dO), which this reproduces); without O_base, the
    kernels' base output is used."""
    out, sel = single_query_decode(cache, layer_id, kv_head, q, seq=seq, page_ids=page_ids, kind=kind,
                                   k_corr_scale=k_corr_scale, score_normalize=score_normalize, router=True,
                                   correction=True, want_diag=True)
    if O_base is None:
        O_base, _ = single_query_decode(cache, layer_id, kv_head, q, seq=seq, page_ids=page_ids, correction=False)
    if debug_stats is not None:
        _debug_accumulate(debug_stats, cache, layer_id, kv_head, seq, page_ids, q, sel, out, O_base, k_corr_scale)
    return out.float() - O_base.float()


def _base_rows(cache: CAREKVCache, layer: int, kv_head: int, page_ids, seq: int):
    """(K_hat, V_hat) fp16 (N, D) of the listed pages' valid rows as the
    decode reads them, and their valid counts."""
    if cache.hat:
        return cache.read_base_hat_concat(layer, kv_head, page_ids, seq=seq)
    from .prefill import dequantize_rows
    kc, ks, vc, vs, lens = cache.read_base_concat(layer, kv_head, page_ids, seq=seq)
    g = cache.cfg.group_size
    return dequantize_rows(kc, ks, g), dequantize_rows(vc, vs, g), lens


def _debug_accumulate(stats: dict, cache: CAREKVCache, layer: int, kv_head: int, seq: int, page_ids, q, sel, out,
                      O_base, k_corr_scale: float) -> None:
    """The debug sums of one corrected query (attention.py:358-372): slots
    read, |dV| of the linear V term sum_t a_t R_V,t over the selected V
    blocks, |k_corr_scale dK| of the linear K term sum_t a_t (q . R_K,t)
    (V_t - O_base) over the selected K groups (attention.py:273-340), |dO|
    of the applied correction and |O_base|; a_t is the fp32 softmax of the
    listed pages' K_hat rows."""
    cfg = cache.cfg
    pids = cache.all_page_ids(layer, kv_head, seq) if page_ids is None else [int(p) for p in page_ids]
    nk = sum(1 for c in sel if c[0] == 0)
    stats["k_slots_read"] = stats.get("k_slots_read", 0) + nk
    stats["v_slots_read"] = stats.get("v_slots_read", 0) + len(sel) - nk
    stats["n_queries"] = stats.get("n_queries", 0) + 1
    D, ps, cg, vb = cfg.head_dim, cfg.page_size, cfg.k_channel_group, cfg.v_token_block
    Kh, Vh, lens = _base_rows(cache, layer, kv_head, pids, seq)
    qf = q.float().reshape(-1)
    a = torch.softmax((Kh.float() @ qf) / math.sqrt(D), dim=0)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    where = {p: i for i, p in enumerate(pids)}
    Ob = O_base.float().reshape(-1)
    dV = torch.zeros(D, dtype=torch.float32, device=q.device)
    dK = torch.zeros_like(dV)
    from .residual import unpack_4bit
    for kind_, page, sub in sel:
        i = where[page]
        p0, n = int(off[i]), int(lens[i])
        if kind_ == 1:
            slot = int(cache.v_slot[layer, kv_head, seq, page, sub])
            R = unpack_4bit(cache.v_res[seq, slot], cache.v_res_scale[seq, slot:slot + 1], vb * D).view(vb, D)
            t0, t1 = sub * vb, min(sub * vb + vb, n)
            if t1 > t0:
                dV += (a[p0 + t0:p0 + t1, None] * R[:t1 - t0]).sum(0)
        else:
            slot = int(cache.k_slot[layer, kv_head, seq, page, sub])
            R = unpack_4bit(cache.k_res[seq, slot], cache.k_res_scale[seq, slot:slot + 1], ps * cg).view(ps, cg)[:n]
            qd = R @ qf[sub * cg:(sub + 1) * cg]
            dK += ((a[p0:p0 + n] * qd)[:, None] * (Vh[p0:p0 + n].float() - Ob)).sum(0)
    stats["delta_v_norm_sum"] = stats.get("delta_v_norm_sum", 0.0) + float(dV.norm())
    stats["delta_k_norm_sum"] = stats.get("delta_k_norm_sum", 0.0) + float((k_corr_scale * dK).norm())
    stats["delta_o_norm_sum"] = stats.get("delta_o_norm_sum", 0.0) + float((out.float().reshape(-1) - Ob).norm())
    stats["o_base_norm_sum"] = stats.get("o_base_norm_sum", 0.0) + float(Ob.norm())


class CAREKVAttention:
    """Per-query-head decode (attention.py:964-1039)."""

    def __init__(self, cfg: CacheConfig, layer_id: int, device=None):
        self.cfg, self.layer_id, self.device = cfg, layer_id, device
        from .residual import ResidualRouter
        self.router = ResidualRouter(cfg, layer_id, device)
        self.scale_factor = 1.0 / math.sqrt(cfg.head_dim)

    def forward(self, cache: CAREKVCache, kv_head: int, q: torch.Tensor, page_ids=None, kind: str = "both",
                k_corr_scale: float = 1.0, score_normalize: bool = False, debug_stats=None, seq: int = 0):
        """Base attention of q over the kv head's pages, corrected through
        the router when ``decode_read_mode`` opens the gate (under
        cfg.compat: read_budget_ratio > 0, attention.py:1025).  (D,) in q's
        dtype; zeros when the kv head holds no page."""
        if cache.num_pages(self.layer_id, kv_head, seq) == 0 or (page_ids is not None and len(page_ids) == 0):
            return torch.zeros(self.cfg.head_dim, dtype=q.dtype, device=q.device)
        gate, knobs = decode_read_mode(self.cfg, self.layer_id)
        corr = gate and kind in ("v", "k", "both")
        out, sel = single_query_decode(cache, self.layer_id, kv_head, q, seq=seq, page_ids=page_ids, kind=kind,
                                       k_corr_scale=k_corr_scale, score_normalize=score_normalize,
                                       router=not knobs.kscore_live, correction=corr,
                                       want_diag=corr and debug_stats is not None)
        if corr and debug_stats is not None:
            O_base, _ = single_query_decode(cache, self.layer_id, kv_head, q, seq=seq, page_ids=page_ids,
                                            correction=False)
            _debug_accumulate(debug_stats, cache, self.layer_id, kv_head, seq, page_ids, q, sel, out, O_base,
                              k_corr_scale)
        return out.to(q.dtype)

    __call__ = forward


class CAREKVMultiHeadAttention:
    """Multi-head decode for one sequence (attention.py:1042-1077)."""

    def __init__(self, cfg: CacheConfig, layer_id: int, device=None):
        assert cfg.num_heads % cfg.num_kv_heads == 0
        self.cfg, self.layer_id, self.device = cfg, layer_id, device
        self.kv_group = cfg.num_heads // cfg.num_kv_heads

    def forward(self, cache: CAREKVCache, Q: torch.Tensor, page_ids=None, kind: str = "both",
                k_corr_scale: float = 1.0, score_normalize: bool = False, debug_stats=None, seq: int = 0,
                correction: Optional[bool] = None):
        """Q (num_heads, D) -> (num_heads, D) fp16.  ``correction=None``: the
        gate and selector of ``decode_read_mode`` (under ``cfg.compat`` the
        reference's: only when read_budget_ratio > 0, attention.py:1025)."""
        cfg = self.cfg
        gate, knobs = decode_read_mode(cfg, self.layer_id)
        knobs.kind = kind
        knobs.k_corr_scale = k_corr_scale
        knobs.normalize = score_normalize
        if correction is None:
            correction = gate
        return decode_attention(cache, self.layer_id, Q.unsqueeze(0), [seq], correction=correction,
                                knobs=knobs)[0]

    __call__ = forward


def single_query_decode(cache: CAREKVCache, layer: int, kv_head: int, q: torch.Tensor, *, seq: int = 0,
                        page_ids=None, kind: str = "both", k_corr_scale: float = 1.0, score_normalize: bool = False,
                        router: bool = True, correction: bool = True, want_diag: bool = False):
    """Decode output of one query vector q (D,) against kv head ``kv_head``
    of sequence ``seq`` (pages ``page_ids`` in list order, default all;
    a list other than 0..n-1 is gathered into a page view first): the
    batched kernels over a one-row batch
    whose other query heads are zero (selection is per query row,
    attention.py:830-875).  ``router``: ResidualRouter.route's sketch-proxy
    score (the per-query reference path); else the knobs of the environment.
    Returns (out (D,) fp16, selected candidate ids [(kind, page, sub)] when
    ``want_diag``)."""
    cfg = cache.cfg
    grp = cfg.num_heads // cfg.num_kv_heads
    n_all = cache.num_pages(layer, kv_head, seq)
    n = n_all if page_ids is None else len(page_ids)
    if page_ids is not None and [int(p) for p in page_ids] != list(range(n)):
        # any other page list: the pages gathered, in list order, into a
        # one-sequence view whose prefix the kernels read
        pids = [int(p) for p in page_ids]
        view = cache.page_view(layer, kv_head, pids, seq=seq)
        out, sel = single_query_decode(view, layer, kv_head, q, seq=0, kind=kind, k_corr_scale=k_corr_scale,
                                       score_normalize=score_normalize, router=router, correction=correction,
                                       want_diag=want_diag)
        return out, (None if sel is None else [(c, pids[p], sub) for c, p, sub in sel])
    knobs = resolve_read_knobs(cfg, layer)
    knobs.kind, knobs.k_corr_scale, knobs.normalize = kind, k_corr_scale, score_normalize
    if router:
        knobs.kscore_live = False
    Q = torch.zeros(1, cfg.num_heads, cfg.head_dim, dtype=torch.float16, device=cache.device)
    h = kv_head * grp
    Q[0, h] = q.to(torch.float16)
    count = correction and debug_stats_enabled()
    diag_cap = (cache.k_cap + cache.v_cap) * max(n, 1) if (want_diag or count) else 0
    # the launch's other (zero) query heads select too: count this query's reads only
    res = decode_attention(cache, layer, Q, [seq], correction=correction, knobs=knobs, n_pages=[n],
                           diag_cap=diag_cap, count_reads=False)
    if not diag_cap:
        return res[0, h], None
    out, diag = res
    sel = _diag_ids(diag[0, h].cpu())
    if count:
        _read_counts_ptr(cache.device)
        nk = sum(1 for c in sel if c[0] == 0)
        _READ_COUNTS[str(cache.device)] += torch.tensor([nk, len(sel) - nk, 1], dtype=torch.int64,
                                                        device=cache.device)
    return out[0, h], (sel if want_diag else None)


def _diag_ids(row) -> list:
    out = []
    for x in row.tolist():
        if x < 0:
            break
        out.append((x >> 30, (x >> 3) & ((1 << 27) - 1), x & 7))
    return out
