"""The reference's store-time and read-time residual classes on the HIP
library: ``ResidualStoreManager`` (residual_store.py:221-464),
``ResidualRouter`` (residual_router.py:79-452) and the 4-bit slot packers
``pack_4bit`` / ``unpack_4bit`` (residual_store.py:121-146).

``process_page`` is one job of ``carekv_store_pages`` with the caller's base
codes and fp16 scales (the page itself was written by ``write_base``), so the
error norms, sketches, prior sort, budgets, ascending slot ids and 4-bit
payloads are those of the prefill store.  ``route`` runs the decode kernels
for its one query with the router's sketch-proxy score and returns the
selection; its scores come from the cache pages (the base logits, weights
and output the reference's callers pass are those of the same pages).
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import numpy as np
import torch
from torch import Tensor

from . import _lib
from .cache import CAREKVCache, PageMeta, get_sketch_proj  # noqa: F401  (get_sketch_proj re-exported)
from .config import CacheConfig, resolve_store_knobs

F16 = torch.float16


def pack_4bit(x: Tensor, scale_hint: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """residual_store.py:121-136: symmetric 4-bit codes of x (s = max|x| / 7
    in x's arithmetic, fp32 or fp16), pairs lo | hi << 4 -> (packed int8
    (ceil(numel / 2),), scale fp16 (1,))."""
    _lib.ptr(x)
    if x.dtype not in (torch.float32, torch.float16):
        raise NotImplementedError(f"pack_4bit of {x.dtype} (fp32 and fp16 are built)")
    x = x.contiguous()
    n = x.numel()
    packed = torch.empty((n + 1) // 2, dtype=torch.int8, device=x.device)
    scale = torch.empty(1, dtype=F16, device=x.device)
    lib = _lib.load()
    _lib.check(lib.carekv_pack_4bit(x.data_ptr(), int(x.dtype == torch.float16), n, packed.data_ptr(),
                                    scale.data_ptr(), _lib.stream_ptr(x.device)), "carekv_pack_4bit")
    return packed, scale


def unpack_4bit(packed: Tensor, scale: Tensor, numel: int) -> Tensor:
    """residual_store.py:139-146: float32 code * float(scale)."""
    _lib.ptr(packed)
    packed = packed.to(torch.int8).contiguous()
    scale = scale.to(F16).contiguous()
    out = torch.empty(numel, dtype=torch.float32, device=packed.device)
    lib = _lib.load()
    _lib.check(lib.carekv_unpack_4bit(packed.data_ptr(), scale.data_ptr(), numel, out.data_ptr(),
                                      _lib.stream_ptr(packed.device)), "carekv_unpack_4bit")
    return out


class ResidualStoreManager:
    """Store-time residual selection for one layer (residual_store.py:221-464)."""

    def __init__(self, cfg: CacheConfig, layer_id: int, device=None):
        self.cfg = cfg
        self.layer_id = layer_id
        self.device = device
        self.sensitivity = cfg.layer_sensitivity[layer_id]

    def process_page(self, cache: CAREKVCache, kv_head: int, page_id: int, K_orig: Tensor, V_orig: Tensor,
                     K_codes: Optional[Tensor], K_scale: Optional[Tensor], V_codes: Optional[Tensor],
                     V_scale: Optional[Tensor], token_start: int, num_valid: int, is_recent: bool = True,
                     is_sink: bool = False, K_hat_override: Optional[Tensor] = None,
                     V_hat_override: Optional[Tensor] = None, seq: int = 0) -> Optional[PageMeta]:
        """residual_store.py:239-464 for one page the caller has written:
        R = half(X_orig - X_hat) with X_hat = half(code * fp16 scale) (or the
        override for a side-buffer base), K candidates per 32-channel group,
        V candidates per 4-token block, the prior sort and budgets, 4-bit
        slots at the next slot ids, the page metadata.  X_orig: (page_size,
        D) rows zero padded past num_valid.  Returns the page's PageMeta."""
        cfg = self.cfg
        T, D = cfg.page_size, cfg.head_dim
        pad = lambda t: torch.nn.functional.pad(t, (0, 0, 0, T - t.shape[0])) if t.shape[0] < T else t  # noqa: E731
        Ko, Vo = pad(K_orig.to(F16)).contiguous(), pad(V_orig.to(F16)).contiguous()
        knobs = resolve_store_knobs(cfg, self.layer_id)
        # the kernel derives is_sink as token_start < sink_tokens
        sink_tokens = int(token_start) + 1 if is_sink else int(token_start)
        sp = _lib.StoreParams(k_budget=knobs.k_budget, v_budget=knobs.v_budget, joint_budget=knobs.joint_budget,
                              joint=int(knobs.joint), store_none=int(knobs.store_none),
                              sensitivity=knobs.sensitivity, sink_tokens=sink_tokens,
                              sketch_proj=cache.sketch_proj.data_ptr())
        keep = []
        if cache.hat:
            if K_hat_override is None or V_hat_override is None:
                raise ValueError("a side-buffer base needs K_hat_override / V_hat_override")
            kh, vh = pad(K_hat_override.to(F16)).contiguous(), pad(V_hat_override.to(F16)).contiguous()
            sp.k_hat, sp.v_hat = kh.data_ptr(), vh.data_ptr()
            keep += [kh, vh]
        else:
            if K_codes is None or K_scale is None or V_codes is None or V_scale is None:
                raise ValueError("a packed base needs K_codes / K_scale / V_codes / V_scale")
            kc, vc = pad(K_codes.to(torch.int8)).contiguous(), pad(V_codes.to(torch.int8)).contiguous()
            ksc, vsc = pad(K_scale.to(F16)).contiguous(), pad(V_scale.to(F16)).contiguous()
            sp.k_codes_in, sp.k_scale_in = kc.data_ptr(), ksc.data_ptr()
            sp.v_codes_in, sp.v_scale_in = vc.data_ptr(), vsc.data_ptr()
            keep += [kc, vc, ksc, vsc]
        for t in [Ko, Vo] + keep:
            _lib.ptr(t)
        jobs = np.array([[seq, kv_head, page_id, num_valid, int(token_start), int(bool(is_recent))]], np.int32)
        jobs_d = torch.from_numpy(jobs).to(cache.device)
        gp = torch.tensor([0, 1], dtype=torch.int32, device=cache.device)
        lib = _lib.load()
        ws = cache.workspace("store", _lib.store_workspace_bytes(lib, cache.arena(self.layer_id), sp, 1))
        _lib.check(lib.carekv_store_pages(cache.arena(self.layer_id), sp, Ko.data_ptr(), Vo.data_ptr(),
                                          jobs_d.data_ptr(), 1, gp.data_ptr(), 1, ws.data_ptr(),
                                          _lib.stream_ptr(cache.device)), "carekv_store_pages (process_page)")
        if _lib.check_enabled():
            _lib.check_status(ws, 4, "carekv_store_pages (process_page)")
        else:
            cache.status.watch(ws, 4, "carekv_store_pages (process_page)")
        cache.valid_host[self.layer_id, kv_head, seq, page_id] = num_valid
        cache._token_start[self.layer_id, kv_head, seq, page_id] = token_start
        return cache.page_meta(self.layer_id, kv_head, page_id, seq)


class ResidualRouter:
    """Read-time routing (residual_router.py:79-452), one query per call."""

    def __init__(self, cfg: CacheConfig, layer_id: int, device=None):
        self.cfg = cfg
        self.layer_id = layer_id
        self.device = device
        self.sensitivity = cfg.layer_sensitivity[layer_id]

    def route(self, cache: CAREKVCache, kv_head: int, page_ids: List[int], q: Tensor, s_base=None, a_base=None,
              O_base=None, V_base_full=None, kind: str = "both", score_normalize: bool = False, debug_stats=None,
              seq: int = 0):
        """residual_router.py:88-452: the stored slots to read for query q
        of kv head ``kv_head`` under cfg's policy and budgets, scored by
        attn_mass * |q_sketch . k_sketch| * boundary * v_diff * sens (K) and
        blk_mass * v_err * sens (V) over pages 0..n-1 of the cache.
        Returns (k_selected [(page, cg, slot)], v_selected [(page, vb, slot)])."""
        from .attention import single_query_decode
        _, sel = single_query_decode(cache, self.layer_id, kv_head, q, seq=seq, page_ids=page_ids, kind=kind,
                                     score_normalize=score_normalize, k_corr_scale=1.0, router=True,
                                     correction=True, want_diag=True)
        k_sel, v_sel = [], []
        ks = cache.k_slot[self.layer_id, kv_head, seq]
        vs = cache.v_slot[self.layer_id, kv_head, seq]
        for kind_, page, sub in sel:
            if kind_ == 0:
                k_sel.append((page, sub, int(ks[page, sub])))
            else:
                v_sel.append((page, sub, int(vs[page, sub])))
        if debug_stats is not None:
            debug_stats["router_n_k_selected"] = debug_stats.get("router_n_k_selected", 0) + len(k_sel)
            debug_stats["router_n_v_selected"] = debug_stats.get("router_n_v_selected", 0) + len(v_sel)
            debug_stats["router_n_route_calls"] = debug_stats.get("router_n_route_calls", 0) + 1
        return k_sel, v_sel
