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
from .cache import CAREKVCache, get_sketch_proj
from .config import CacheConfig, ReadKnobs, resolve_read_knobs

KIND_CODE = {"both": 0, "k": 1, "v": 2}


def default_split_pages(max_pages: int, rows: int) -> int:
    """Pages per work-group: enough work-groups to fill 256 CUs several times
    over, and a multiple of 16 (4 waves x 4-page windows)."""
    target = int(os.environ.get("CAREKV_DECODE_TARGET_WGS", "4096"))
    sp = math.ceil(max(1, max_pages) * max(1, rows) / target)
    sp = max(16, min(256, sp))
    return (sp + 15) // 16 * 16


def decode_attention(cache: CAREKVCache, layer: int, q: torch.Tensor, seqs: Optional[Sequence[int]] = None, *,
                     correction: bool = True, knobs: Optional[ReadKnobs] = None, split_pages: Optional[int] = None,
                     diag_cap: int = 0, out: Optional[torch.Tensor] = None, phase_events=None):
    """q: (B, Hq, D) fp16 post-RoPE queries of B sequences -> (B, Hq, D) fp16.

    With ``diag_cap > 0`` also returns the selected candidates per query
    head as an int32 (B, Hq, diag_cap) tensor (kind<<30 | page<<3 | sub, -1
    padded), for parity checks.  ``phase_events``: optional sequence of 5
    recorded torch.cuda.Event (timing enabled), re-recorded on the launch
    stream around the streaming, select, apply and combine kernels."""
    cfg: CacheConfig = cache.cfg
    if q.dim() == 2:
        q = q.unsqueeze(0)
    B, Hq, D = q.shape
    assert D == cfg.head_dim and Hq == cfg.num_heads
    seqs = list(range(B)) if seqs is None else list(seqs)
    if knobs is None:
        knobs = resolve_read_knobs(cfg, layer)
    q = q.to(torch.float16).contiguous()
    npages = np.array([cache.num_pages(layer, 0, s) for s in seqs], dtype=np.int32)
    max_np = int(npages.max()) if B else 0
    dev = cache.device
    key = (tuple(seqs), npages.tobytes())
    meta = cache._row_tables.get(key)
    if meta is None:  # device row table, reused while the batch is unchanged
        meta = torch.from_numpy(np.stack([np.array(seqs, dtype=np.int32), npages])).to(dev)
        if len(cache._row_tables) > 64:
            cache._row_tables.clear()
        cache._row_tables[key] = meta
    if split_pages is None:
        split_pages = default_split_pages(max_np, B * cfg.num_kv_heads)
    dp = _lib.DecodeParams(
        batch=B, n_heads=Hq, seq_slot=meta[0].data_ptr(), n_pages=meta[1].data_ptr(), max_pages_used=max_np,
        sm_scale=float(np.float32(1.0 / math.sqrt(D))), sensitivity=float(cfg.layer_sensitivity[layer]),
        correction=int(bool(correction)), kind=KIND_CODE[knobs.kind], joint=int(knobs.joint),
        normalize=int(knobs.normalize), k_exact=int(knobs.k_exact), k_corr_scale=knobs.k_corr_scale,
        lambda_k=knobs.lambda_k, lambda_v=knobs.lambda_v, budget_ratio=int(knobs.budget_ratio),
        abs_k=knobs.abs_k, abs_v=knobs.abs_v, ratio_k=knobs.ratio_k, ratio_v=knobs.ratio_v,
        k_cap=cache.k_cap, v_cap=cache.v_cap, split_pages=int(split_pages),
        route_policy=int(knobs.route_policy), adaptive_score=int(bool(knobs.adaptive_score)),
        rel_threshold=float(knobs.rel_threshold), abs_threshold=float(knobs.abs_threshold),
        min_keep=int(knobs.min_keep))
    if correction and not knobs.kscore_live:
        P = get_sketch_proj(cfg.head_dim, cfg.k_channel_group, cfg.sketch_dim, dev)
        dp.k_proxy = 1
        dp.sketch_proj = P.data_ptr()
    ev_arr = None
    if phase_events is not None:
        if len(phase_events) != 5:
            raise ValueError("phase_events needs 5 events")
        ev_arr = (ctypes.c_void_p * 5)(*[int(e.cuda_event) for e in phase_events])
        dp.phase_events = ctypes.cast(ev_arr, ctypes.c_void_p)
    lib = _lib.load()
    a = cache.arena(layer)
    nbytes = int(lib.carekv_decode_workspace_bytes(a, dp))
    if nbytes < 0:
        raise _lib.CarekvError("carekv_decode_workspace_bytes rejected the parameters")
    ws = cache.workspace("decode", nbytes)
    if out is None:
        out = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)
    diag = torch.empty(B, Hq, diag_cap, dtype=torch.int32, device=dev) if diag_cap > 0 else None
    _lib.check(lib.carekv_decode_attn(a, dp, q.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                      None if diag is None else diag.data_ptr(), int(diag_cap),
                                      _lib.stream_ptr(dev)), "carekv_decode_attn")
    return (out, diag) if diag_cap > 0 else out


class CAREKVMultiHeadAttention:
    """Multi-head decode for one sequence (attention.py:1042-1077)."""

    def __init__(self, cfg: CacheConfig, layer_id: int, device=None):
        assert cfg.num_heads % cfg.num_kv_heads == 0
        self.cfg, self.layer_id, self.device = cfg, layer_id, device
        self.kv_group = cfg.num_heads // cfg.num_kv_heads

    def forward(self, cache: CAREKVCache, Q: torch.Tensor, page_ids=None, kind: str = "both",
                k_corr_scale: float = 1.0, score_normalize: bool = False, debug_stats=None, seq: int = 0,
                correction: Optional[bool] = None):
        """Q (num_heads, D) -> (num_heads, D) fp16.  The reference applies its
        correction only when read_budget_ratio > 0 (attention.py:1025);
        ``correction=None`` keeps that gate."""
        cfg = self.cfg
        knobs = resolve_read_knobs(cfg, self.layer_id)
        knobs.kind = kind
        knobs.k_corr_scale = k_corr_scale
        knobs.normalize = score_normalize
        if correction is None:
            correction = cfg.read_budget_ratio > 0
        return decode_attention(cache, self.layer_id, Q.unsqueeze(0), [seq], correction=correction,
                                knobs=knobs)[0]

    __call__ = forward
