"""Paged cache restatement (``cache.py:209-904``) in numpy.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from . import quant as Q

F16, F32 = np.float16, np.float32


@dataclass
class OCfg:
    """Subset of ``CacheConfig`` (``cache.py:209-375``) the hot path reads."""
    num_layers: int = 1
    num_heads: int = 32
    num_kv_heads: Optional[int] = None
    head_dim: int = 128
    page_size: int = 16
    max_pages: int = 512
    base_bits: int = 3
    residual_bits: int = 4
    group_size: int = 32
    k_channel_group: int = 32
    v_token_block: int = 4
    store_budget_ratio: float = 0.0
    read_budget_ratio: float = 0.0
    sketch_dim: int = 32
    layer_sensitivity: Optional[List[float]] = None
    packed_base: bool = True
    scale_quant: str = "int8"
    store_budget_mode: str = "absolute"
    read_budget_mode: str = "absolute"
    store_budget_ratio_k: Optional[float] = None
    store_budget_ratio_v: Optional[float] = None
    read_budget_ratio_k: Optional[float] = None
    read_budget_ratio_v: Optional[float] = None
    store_abs_k: int = 0
    store_abs_v: int = 0
    read_abs_k: int = 0
    read_abs_v: int = 0
    route_policy: str = "joint"
    budget_policy: str = "uniform"
    read_relative_threshold: float = 0.0
    read_absolute_threshold: float = 0.0
    read_min_keep: int = 0
    base_quantizer: str = "uniform"
    k_bits_override: int = -1
    v_bits_override: int = -1

    @property
    def side_buffer(self) -> bool:
        """fp16 K_hat / V_hat side buffer (cache.py:487-499; the decode read
        checks these three names, attention.py:997)."""
        return self.base_quantizer in ("kivi_style", "rotatekv_style", "kvquant_style")

    def kivi_bits(self):
        """``layer.py:197-202``."""
        kb = self.k_bits_override if self.k_bits_override > 0 else self.base_bits
        vb = self.v_bits_override if self.v_bits_override > 0 else self.base_bits
        return int(kb), int(vb)

    def __post_init__(self):
        if self.layer_sensitivity is None:
            self.layer_sensitivity = [1.0] * self.num_layers
        if self.num_kv_heads is None:
            self.num_kv_heads = self.num_heads


def layer_budget_multiplier(cfg: OCfg, layer_id: int) -> float:
    """``cache.py:166-202``."""
    L = cfg.num_layers
    if cfg.budget_policy == "uniform" or L <= 1:
        return 1.0
    if cfg.budget_policy == "u_shaped":
        raw = [0.5 + 1.5 * abs(2 * (l / (L - 1)) - 1) for l in range(L)]
        m = sum(raw) / L
        return raw[layer_id] / m
    if cfg.budget_policy == "sensitivity":
        s = cfg.layer_sensitivity or [1.0] * L
        ms = sum(s) / max(L, 1)
        return 1.0 if ms <= 0 else s[layer_id] / ms
    return 1.0


@dataclass
class OMeta:
    """``PageMeta`` (``cache.py:391-409``)."""
    page_id: int
    layer_id: int
    kv_head: int
    token_start: int
    num_tokens: int
    k_residual_slots: List[int] = field(default_factory=list)
    v_residual_slots: List[int] = field(default_factory=list)
    k_error_norm: Optional[np.ndarray] = None
    v_error_norm: Optional[np.ndarray] = None
    k_sketch: Optional[np.ndarray] = None
    prior_score: float = 0.0


class OCache:
    """``CAREKVCache`` restated for packed_base + scale_quant in {none,int8}."""

    def __init__(self, cfg: OCfg, max_slots: Optional[int] = None):
        self.cfg = cfg
        L, H, P, T, D = cfg.num_layers, cfg.num_kv_heads, cfg.max_pages, cfg.page_size, cfg.head_dim
        G = D // cfg.group_size
        rb = Q.packed_row_bytes(D, cfg.base_bits) if cfg.packed_base else D
        self.base_K_codes = np.zeros((L, H, P, T, rb), np.int8)
        self.base_V_codes = np.zeros((L, H, P, T, rb), np.int8)
        if cfg.scale_quant == "int8":
            self.base_K_scale = np.zeros((L, H, P, T, G), np.int8)
            self.base_V_scale = np.zeros((L, H, P, T, G), np.int8)
            self.base_K_scale_master = np.zeros((L, H, P), F16)
            self.base_V_scale_master = np.zeros((L, H, P), F16)
        else:
            self.base_K_scale = np.zeros((L, H, P, T, G), F16)
            self.base_V_scale = np.zeros((L, H, P, T, G), F16)
            self.base_K_scale_master = self.base_V_scale_master = None
        self.valid_tokens = np.zeros((L, H, P), np.int32)
        if cfg.side_buffer:                                     # cache.py:487-499
            self.base_K_hat_fp16 = np.zeros((L, H, P, T, D), F16)
            self.base_V_hat_fp16 = np.zeros((L, H, P, T, D), F16)
        else:
            self.base_K_hat_fp16 = self.base_V_hat_fp16 = None
        self.open_rows = {}  # (layer, kv head, page) -> true K / V rows of an open page (streaming store)
        self.open_scales = {}  # (layer, kv head, page) -> fp16 group scales of an open page's rows (re-encoding)
        if max_slots is None:                                   # cache.py:507-509
            ratio_est = int(P * H * L * cfg.store_budget_ratio * 4)
            abs_est = int(P * H * L * (cfg.store_abs_k + cfg.store_abs_v) * 2)
            max_slots = max(64, ratio_est, abs_est)
        rbits = cfg.residual_bits
        self.k_slot_bytes = T * cfg.k_channel_group * rbits // 8
        self.v_slot_bytes = cfg.v_token_block * D * rbits // 8
        self.k_residual_buf = np.zeros((max_slots, self.k_slot_bytes), np.int8)
        self.v_residual_buf = np.zeros((max_slots, self.v_slot_bytes), np.int8)
        self.k_residual_scale = np.zeros((max_slots, 1), F16)
        self.v_residual_scale = np.zeros((max_slots, 1), F16)
        self.next_k_slot = 0          # pop(0) of an ascending free list (cache.py:548-560)
        self.next_v_slot = 0
        self.meta_table = [[[None] * P for _ in range(H)] for _ in range(L)]
        self.next_page = [[0] * H for _ in range(L)]

    # -- allocation (cache.py:542-566)
    def alloc_page(self, layer, kv_head):
        pid = self.next_page[layer][kv_head]
        assert pid < self.cfg.max_pages, "KV cache is full"
        self.next_page[layer][kv_head] += 1
        return pid

    def alloc_k_slot(self):
        assert self.next_k_slot < self.k_residual_buf.shape[0], "K residual buffer is full"
        s = self.next_k_slot
        self.next_k_slot += 1
        return s

    def alloc_v_slot(self):
        assert self.next_v_slot < self.v_residual_buf.shape[0], "V residual buffer is full"
        s = self.next_v_slot
        self.next_v_slot += 1
        return s

    def get_open_page(self, layer, kv_head):
        """``cache.py:572-583``."""
        n = self.next_page[layer][kv_head]
        if n == 0:
            return None
        last = n - 1
        return last if int(self.valid_tokens[layer, kv_head, last]) < self.cfg.page_size else None

    def all_page_ids(self, layer, kv_head):
        return list(range(self.next_page[layer][kv_head]))

    def total_valid_tokens(self, layer, kv_head):
        n = self.next_page[layer][kv_head]
        return int(self.valid_tokens[layer, kv_head, :n].sum()) if n else 0

    # -- base write (cache.py:617-701)
    def _write_scale(self, dst_scale, dst_master, idx, scale_in):
        if self.cfg.scale_quant == "int8":
            codes, master = Q.write_scale_page(scale_in)
            dst_scale[idx] = codes
            dst_master[idx] = master
        else:
            dst_scale[idx] = np.asarray(scale_in).astype(F16)

    def write_base(self, layer, kv_head, page_id, K_codes, K_scale, V_codes, V_scale, num_valid):
        cfg = self.cfg
        assert 0 <= num_valid <= cfg.page_size
        idx = (layer, kv_head, page_id)
        if cfg.packed_base:
            self.base_K_codes[idx] = Q.pack_codes_2d(K_codes, cfg.base_bits)
            self.base_V_codes[idx] = Q.pack_codes_2d(V_codes, cfg.base_bits)
        else:
            self.base_K_codes[idx] = K_codes
            self.base_V_codes[idx] = V_codes
        self._write_scale(self.base_K_scale, self.base_K_scale_master, idx, K_scale)
        self._write_scale(self.base_V_scale, self.base_V_scale_master, idx, V_scale)
        self.valid_tokens[idx] = num_valid

    def append_to_page(self, layer, kv_head, page_id, K_codes_row, K_scale_row, V_codes_row, V_scale_row):
        cfg = self.cfg
        off = int(self.valid_tokens[layer, kv_head, page_id])
        assert off < cfg.page_size, "page already full"
        idx = (layer, kv_head, page_id, off)
        if cfg.packed_base:
            self.base_K_codes[idx] = Q.pack_codes_2d(np.asarray(K_codes_row)[None], cfg.base_bits)[0]
            self.base_V_codes[idx] = Q.pack_codes_2d(np.asarray(V_codes_row)[None], cfg.base_bits)[0]
        else:
            self.base_K_codes[idx] = K_codes_row
            self.base_V_codes[idx] = V_codes_row
        if cfg.scale_quant == "int8":
            self.base_K_scale[idx] = Q.append_scale_codes(K_scale_row, self.base_K_scale_master[layer, kv_head, page_id])
            self.base_V_scale[idx] = Q.append_scale_codes(V_scale_row, self.base_V_scale_master[layer, kv_head, page_id])
        else:
            self.base_K_scale[idx] = np.asarray(K_scale_row).astype(F16)
            self.base_V_scale[idx] = np.asarray(V_scale_row).astype(F16)
        self.valid_tokens[layer, kv_head, page_id] = off + 1
        return off

    # -- fp16 side buffer (cache.py:800-865)
    def write_base_kivi(self, layer, kv_head, page_id, K_hat, V_hat, num_valid):
        assert self.base_K_hat_fp16 is not None and 0 <= num_valid <= self.cfg.page_size
        self.base_K_hat_fp16[layer, kv_head, page_id] = np.asarray(K_hat).astype(F16)
        self.base_V_hat_fp16[layer, kv_head, page_id] = np.asarray(V_hat).astype(F16)
        self.valid_tokens[layer, kv_head, page_id] = num_valid

    def append_to_page_kivi(self, layer, kv_head, page_id, K_hat_row, V_hat_row):
        off = int(self.valid_tokens[layer, kv_head, page_id])
        assert off < self.cfg.page_size, "page already full"
        self.base_K_hat_fp16[layer, kv_head, page_id, off] = np.asarray(K_hat_row).astype(F16)
        self.base_V_hat_fp16[layer, kv_head, page_id, off] = np.asarray(V_hat_row).astype(F16)
        self.valid_tokens[layer, kv_head, page_id] = off + 1
        return off

    def read_base_hat_concat(self, layer, kv_head, page_ids):
        Kh, Vh, lens = [], [], []
        for pid in page_ids:
            n = int(self.valid_tokens[layer, kv_head, pid])
            lens.append(n)
            if n == 0:
                continue
            Kh.append(self.base_K_hat_fp16[layer, kv_head, pid, :n])
            Vh.append(self.base_V_hat_fp16[layer, kv_head, pid, :n])
        if not Kh:
            e = np.zeros((0, self.cfg.head_dim), F16)
            return e, e, lens
        return np.concatenate(Kh), np.concatenate(Vh), lens

    # -- base read (cache.py:707-772)
    def unpack_rows(self, rows):
        cfg = self.cfg
        if cfg.packed_base and rows.shape[0] > 0:
            return Q.unpack_codes_2d(rows, cfg.base_bits, cfg.head_dim)
        return rows

    def page_scales(self, layer, kv_head, pid, which, n=None):
        sc = self.base_K_scale if which == "K" else self.base_V_scale
        ms = self.base_K_scale_master if which == "K" else self.base_V_scale_master
        rows = sc[layer, kv_head, pid] if n is None else sc[layer, kv_head, pid, :n]
        if self.cfg.scale_quant == "int8":
            return Q.read_scale(rows, ms[layer, kv_head, pid])
        return rows.astype(F16)

    def read_base_concat(self, layer, kv_head, page_ids):
        cfg = self.cfg
        Kc, Ks, Vc, Vs, lens = [], [], [], [], []
        for pid in page_ids:
            n = int(self.valid_tokens[layer, kv_head, pid])
            lens.append(n)
            if n == 0:
                continue
            Kc.append(self.unpack_rows(self.base_K_codes[layer, kv_head, pid, :n]))
            Vc.append(self.unpack_rows(self.base_V_codes[layer, kv_head, pid, :n]))
            Ks.append(self.page_scales(layer, kv_head, pid, "K", n))
            Vs.append(self.page_scales(layer, kv_head, pid, "V", n))
        D, G = cfg.head_dim, cfg.head_dim // cfg.group_size
        if not Kc:
            e8, ef = np.zeros((0, D), np.int8), np.zeros((0, G), F16)
            return e8, ef, e8, ef, lens
        return (np.concatenate(Kc), np.concatenate(Ks), np.concatenate(Vc), np.concatenate(Vs), lens)

    # -- residual slots (cache.py:871-883)
    def write_k_residual(self, slot, packed, scale):
        self.k_residual_buf[slot] = np.asarray(packed).ravel()
        self.k_residual_scale[slot] = scale

    def write_v_residual(self, slot, packed, scale):
        self.v_residual_buf[slot] = np.asarray(packed).ravel()
        self.v_residual_scale[slot] = scale
