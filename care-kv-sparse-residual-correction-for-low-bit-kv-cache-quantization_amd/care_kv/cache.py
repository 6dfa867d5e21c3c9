"""Paged CARE-KV cache on the device.

``CAREKVCache`` keeps the reference's interface (cache.py:416-904): per
(layer, kv head) page counters, ``alloc_page`` / ``get_open_page`` /
``all_page_ids`` / ``read_base_concat`` / ``meta_table`` / slot arenas.  Its
storage is one device arena per model sized for ``n_seq`` sequence slots, so
a batch of sequences is decoded by one kernel launch per layer; with
``n_seq=1`` it is a drop-in for the reference's one-cache-per-sequence object
and its buffer attributes have the reference shapes.

Memory layout (all device tensors):
  base codes   int8 [L, Hkv, n_seq, P, T, row_bytes]  (always bit-packed)
  base scales  int8 [L, Hkv, n_seq, P, T, G] + fp16 master [L, Hkv, n_seq, P]
               (scale_quant=int8) or fp16 [L, Hkv, n_seq, P, T, G]
  page meta    valid/has_meta/k_slot/v_slot/k_err/v_err/k_sketch/v_sq per page
  slot arenas  int8 [n_seq, S, slot_bytes] + fp16 scales, shared by layers
Page counters and valid counts are mirrored on the host (they evolve
deterministically), so appends and decode never read device memory back.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from .config import CacheConfig, resolve_store_knobs, store_caps

F16 = torch.float16


@dataclass
class PageMeta:
    """Per-page metadata (same fields as the reference PageMeta)."""
    page_id: int
    layer_id: int
    kv_head: int
    token_start: int
    num_tokens: int
    k_residual_slots: List[int] = field(default_factory=list)
    v_residual_slots: List[int] = field(default_factory=list)
    k_error_norm: Optional[torch.Tensor] = None
    v_error_norm: Optional[torch.Tensor] = None
    k_sketch: Optional[torch.Tensor] = None
    prior_score: float = 0.0


def to_device(arr: np.ndarray, device) -> torch.Tensor:
    """A host array on the device without waiting for the stream: the bytes
    go through a fresh pinned buffer, which torch's caching host allocator
    keeps until the asynchronous copy has run.  A pageable copy would wait
    for every kernel queued before it, so that the host could not run ahead
    of the GPU in a decode loop."""
    t = torch.from_numpy(np.ascontiguousarray(arr))
    if torch.device(device).type != "cuda":
        return t.to(device, copy=True)
    return t.pin_memory().to(device, non_blocking=True)


def packed_row_bytes(D: int, bits: int) -> int:
    if bits == 2 and D % 4 == 0:
        return D // 4
    if bits == 3 and D % 8 == 0:
        return D * 3 // 8
    if bits == 4 and D % 2 == 0:
        return D // 2
    raise ValueError(f"Unsupported base_bits={bits} for head_dim={D}")


_SKETCH_CACHE: Dict[Tuple[int, int, str], torch.Tensor] = {}


def get_sketch_proj(head_dim: int, k_channel_group: int, sketch_dim: int, device) -> torch.Tensor:
    """Fixed random projection (kcg, sketch_dim): randn from a CPU generator
    seeded 42, divided by sqrt(sketch_dim) (residual_store.py:206-214)."""
    key = (k_channel_group, sketch_dim, str(device))
    if key not in _SKETCH_CACHE:
        gen = torch.Generator(device="cpu").manual_seed(42)
        P = torch.randn(k_channel_group, sketch_dim, generator=gen) / math.sqrt(sketch_dim)
        _SKETCH_CACHE[key] = P.to(device)
    return _SKETCH_CACHE[key]


# Base quantizers whose pages hold fp16 K_hat / V_hat (the side buffer of
# cache.py:487-499) and that the kernels implement: per-channel K / per-token
# V (kivi_helpers.py:35-59; kvquant_style post-RoPE is the same quantizer).
HAT_QUANTIZERS = ("kivi_style", "kvquant_style")


def hat_bits(cfg: CacheConfig) -> Tuple[int, int]:
    """``CAREKVLayer._kivi_bits`` (layer.py:197-202)."""
    kb = cfg.k_bits_override if cfg.k_bits_override > 0 else cfg.base_bits
    vb = cfg.v_bits_override if cfg.v_bits_override > 0 else cfg.base_bits
    return int(kb), int(vb)


def check_kernel_config(cfg: CacheConfig):
    """Configurations the HIP kernels implement; anything else is rejected."""
    bad = []
    if cfg.base_quantizer not in ("uniform",) + HAT_QUANTIZERS:
        bad.append(f"base_quantizer={cfg.base_quantizer} (uniform, kivi_style or kvquant_style post-RoPE)")
    if cfg.base_quantizer == "kvquant_style" and getattr(cfg, "k_store_mode", "post_rope") != "post_rope":
        bad.append("kvquant_style with k_store_mode=pre_rope (post_rope only)")
    if cfg.page_size != 16:
        bad.append(f"page_size={cfg.page_size} (16)")
    if cfg.group_size != 32:
        bad.append(f"group_size={cfg.group_size} (32)")
    if cfg.k_channel_group != 32:
        bad.append(f"k_channel_group={cfg.k_channel_group} (32)")
    if cfg.v_token_block != 4:
        bad.append(f"v_token_block={cfg.v_token_block} (4)")
    if cfg.head_dim not in (64, 128):
        bad.append(f"head_dim={cfg.head_dim} (64 or 128)")
    if cfg.base_bits not in (2, 3, 4):
        bad.append(f"base_bits={cfg.base_bits} (2, 3 or 4)")
    if cfg.residual_bits != 4:
        bad.append(f"residual_bits={cfg.residual_bits} (4)")
    if cfg.scale_quant == "none" and cfg.scale_dtype != "fp16":
        bad.append(f"scale_dtype={cfg.scale_dtype} with scale_quant=none (fp16)")
    if cfg.sketch_dim > 64:
        bad.append(f"sketch_dim={cfg.sketch_dim} (<= 64)")
    if bad:
        raise NotImplementedError("CARE-KV HIP kernels do not support: " + "; ".join(bad))


def kivi_qdq(x: torch.Tensor, bits: int, per_channel: bool) -> torch.Tensor:
    """``quant_dequant_kivi_k`` (per_channel: one scale per channel over the
    rows) / ``quant_dequant_kivi_v`` (one scale per row) of kivi_helpers.py:35-59
    on an fp16 device tensor (..., T, D), through carekv_kivi_qdq."""
    _lib.ptr(x)  # a device tensor, or CarekvError
    x = x.to(F16).contiguous()
    T, D = x.shape[-2], x.shape[-1]
    n_mat = x.numel() // max(T * D, 1)
    out = torch.empty_like(x)
    lib = _lib.load()
    _lib.check(lib.carekv_kivi_qdq(x.data_ptr(), n_mat, T, D, int(bits), int(per_channel), out.data_ptr(),
                                   _lib.stream_ptr(x.device)), "carekv_kivi_qdq")
    return out


def kivi_codes(x: torch.Tensor, bits: int, per_channel: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """The codes and scales behind ``kivi_qdq`` (carekv_kivi_codes; no
    reference counterpart): x fp16 (..., T, D) -> int8 codes (..., T, D) and
    fp16 scales (..., D) per channel or (..., T) per token, NaN where the
    max |x| is 0, so that half(code * scale) is kivi_qdq's output."""
    _lib.ptr(x)
    x = x.to(F16).contiguous()
    T, D = x.shape[-2], x.shape[-1]
    n_mat = x.numel() // max(T * D, 1)
    codes = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scale = torch.empty(x.shape[:-2] + ((D,) if per_channel else (T,)), dtype=F16, device=x.device)
    lib = _lib.load()
    _lib.check(lib.carekv_kivi_codes(x.data_ptr(), n_mat, T, D, int(bits), int(per_channel), codes.data_ptr(),
                                     scale.data_ptr(), _lib.stream_ptr(x.device)), "carekv_kivi_codes")
    return codes, scale


class CAREKVCache:
    """Device-resident paged cache for ``n_seq`` sequences of one model."""

    def __init__(self, cfg: CacheConfig, device=None, n_seq: int = 1, n_slots: Optional[int] = None,
                 streaming_store: Optional[bool] = None):
        """``streaming_store`` (no reference counterpart): keep
        each open page's true fp16 rows and, when decode appends fill the
        page, store its residuals against the page's own base instead of
        the reference's zero-residual fill store (layer.py:1128-1146), so
        that decode-filled pages get slots.  None: on unless ``cfg.compat``.

        Unless ``cfg.compat``, decode appends into int8-scale pages re-encode
        the open page as write_base encodes its valid rows (the fp16 group
        scales of every open page are kept for that) instead of the
        reference's fixed-master encoding, whose decode-opened pages read back
        as zero (cache.py:689-695)."""
        check_kernel_config(cfg)
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.cfg = cfg
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise _lib.CarekvError("CAREKVCache lives on a HIP device (got %s)" % self.device)
        self.n_seq = n_seq
        L, H, P, T, D = cfg.num_layers, cfg.num_kv_heads, cfg.max_pages, cfg.page_size, cfg.head_dim
        G = D // cfg.group_size
        self.ncg = D // cfg.k_channel_group
        self.nvb = math.ceil(T / cfg.v_token_block)
        self.hat = cfg.base_quantizer in HAT_QUANTIZERS  # K_hat / V_hat of the KIVI-style quant-dequant
        # the packed KIVI base (no reference counterpart): 2-bit prompt pages,
        # fp16 K_hat / V_hat only for the later rows
        self.kivi_packed = self.hat and bool(getattr(cfg, "kivi_packed", False))
        if self.kivi_packed and hat_bits(cfg) != (2, 2):
            raise NotImplementedError(f"kivi_packed is built for the 2-bit KIVI base (got K/V bits {hat_bits(cfg)})")
        if self.kivi_packed and cfg.num_heads // cfg.num_kv_heads > 4:
            raise NotImplementedError("kivi_packed decodes with at most 4 query heads per kv head")
        self._arena_bits = 2 if self.kivi_packed else (16 if self.hat else cfg.base_bits)
        self._packed_row_bytes = (2 * D if self.hat and not self.kivi_packed
                                  else packed_row_bytes(D, self._arena_bits))
        dev = self.device
        shp = (L, H, n_seq, P)
        self.kcodes = torch.zeros(*shp, T, self._packed_row_bytes, dtype=torch.int8, device=dev)
        self.vcodes = torch.zeros_like(self.kcodes)
        self.scale_mode = 1 if cfg.scale_quant == "int8" and not self.kivi_packed else 0
        if self.kivi_packed:
            self.tail_pages = int(cfg.kivi_tail_pages) if cfg.kivi_tail_pages > 0 else P
            self.kchan = torch.zeros(L, H, n_seq, D, dtype=F16, device=dev)  # per-channel K scales of the prompt
            self.tail_k = torch.zeros(L, H, n_seq, self.tail_pages, T, D, dtype=F16, device=dev)
            self.tail_v = torch.zeros_like(self.tail_k)
            self.n_packed = np.zeros(n_seq, dtype=np.int32)  # packed prompt pages per sequence
            self.n_packed_d = torch.zeros(n_seq, dtype=torch.int32, device=dev)
        sdt = torch.int8 if self.scale_mode else F16
        self.kscale = torch.zeros(*shp, T, G, dtype=sdt, device=dev)
        self.vscale = torch.zeros_like(self.kscale)
        self.kmaster = torch.zeros(*shp, dtype=F16, device=dev)
        self.vmaster = torch.zeros_like(self.kmaster)
        self.valid = torch.zeros(*shp, dtype=torch.int32, device=dev)
        self.has_meta = torch.zeros(*shp, dtype=torch.int8, device=dev)
        self.k_slot = torch.full((*shp, self.ncg), -1, dtype=torch.int32, device=dev)
        self.v_slot = torch.full((*shp, self.nvb), -1, dtype=torch.int32, device=dev)
        self.k_err = torch.zeros(*shp, self.ncg, dtype=F16, device=dev)
        self.v_err = torch.zeros(*shp, self.nvb, dtype=F16, device=dev)
        self.k_sketch = torch.zeros(*shp, self.ncg, cfg.sketch_dim, dtype=F16, device=dev)
        self.v_sq = torch.zeros(*shp, dtype=torch.float32, device=dev)
        self.streaming_store = (not cfg.compat) if streaming_store is None else bool(streaming_store)
        # open pages' fp16 group scales, for the re-encoding append
        self.rescale_open = self.scale_mode == 1 and not self.hat and not cfg.compat
        if self.rescale_open:
            self.open_ks = torch.zeros(L, H, n_seq, T, G, dtype=F16, device=dev)
            self.open_vs = torch.zeros_like(self.open_ks)
        if self.streaming_store:
            # true rows of every (layer, seq, kv head)'s open page
            self.open_k = torch.zeros(L, n_seq, H, T, D, dtype=F16, device=dev)
            self.open_v = torch.zeros_like(self.open_k)
        self.k_cap, self.v_cap = store_caps(cfg)
        if n_slots is None:
            n_slots = max(64, P * H * L * self.k_cap, P * H * L * self.v_cap)
            if self.streaming_store:  # the prompt's partial last page is stored twice (prefill, then on fill)
                n_slots += L * H * max(self.k_cap, self.v_cap)
        self.n_slots = n_slots
        self.k_slot_bytes = T * cfg.k_channel_group * cfg.residual_bits // 8
        self.v_slot_bytes = cfg.v_token_block * D * cfg.residual_bits // 8
        self.k_res = torch.zeros(n_seq, n_slots, self.k_slot_bytes, dtype=torch.int8, device=dev)
        self.v_res = torch.zeros(n_seq, n_slots, self.v_slot_bytes, dtype=torch.int8, device=dev)
        self.k_res_scale = torch.zeros(n_seq, n_slots, dtype=F16, device=dev)
        self.v_res_scale = torch.zeros(n_seq, n_slots, dtype=F16, device=dev)
        self.next_slot = torch.zeros(n_seq, 2, dtype=torch.int32, device=dev)
        self.sketch_proj = get_sketch_proj(D, cfg.k_channel_group, cfg.sketch_dim, dev).contiguous()
        # host mirrors
        self.next_page = np.zeros((L, H, n_seq), dtype=np.int64)
        self.valid_host = np.zeros((L, H, n_seq, P), dtype=np.int32)
        self._token_start = np.zeros((L, H, n_seq, P), dtype=np.int64)
        self._arenas: Dict[int, _lib.Arena] = {}
        self._freed: Dict[Tuple[int, int], List[int]] = {}  # (seq, 0 K / 1 V) -> freed slot ids
        self._ws: Dict[str, torch.Tensor] = {}
        self._row_tables: Dict[tuple, torch.Tensor] = {}
        self.status = _lib.StatusWatch()  # store calls' slot-overflow words, read without a sync
        # optional (start, end) torch.cuda.Event pair that write_prefill records
        # on the stream right before and after its store launches
        self.store_events = None
        _lib.load()

    # ------------------------------------------------------------ C structs
    def arena(self, layer: int) -> _lib.Arena:
        a = self._arenas.get(layer)
        if a is None:
            cfg = self.cfg
            g = lambda t: t[layer].data_ptr()  # noqa: E731
            a = _lib.Arena(
                kcodes=g(self.kcodes), vcodes=g(self.vcodes), kscale=g(self.kscale), vscale=g(self.vscale),
                kmaster=g(self.kmaster), vmaster=g(self.vmaster), valid=g(self.valid), has_meta=g(self.has_meta),
                k_slot=g(self.k_slot), v_slot=g(self.v_slot), k_err=g(self.k_err), v_err=g(self.v_err),
                k_sketch=g(self.k_sketch), v_sq=g(self.v_sq), k_res=self.k_res.data_ptr(),
                k_res_scale=self.k_res_scale.data_ptr(), v_res=self.v_res.data_ptr(),
                v_res_scale=self.v_res_scale.data_ptr(), next_slot=self.next_slot.data_ptr(),
                n_seq=self.n_seq, n_kv_heads=cfg.num_kv_heads, max_pages=cfg.max_pages, head_dim=cfg.head_dim,
                base_bits=self._arena_bits, page_size=cfg.page_size, group_size=cfg.group_size,
                k_channel_group=cfg.k_channel_group, v_token_block=cfg.v_token_block, sketch_dim=cfg.sketch_dim,
                scale_mode=self.scale_mode, residual_bits=cfg.residual_bits, n_slots=self.n_slots,
                hat_bits_k=hat_bits(cfg)[0], hat_bits_v=hat_bits(cfg)[1],
                open_kscale=g(self.open_ks) if self.rescale_open else None,
                open_vscale=g(self.open_vs) if self.rescale_open else None, rescale_open=int(self.rescale_open),
                streaming_store=int(self.streaming_store))
            if self.kivi_packed:
                a.kivi_packed = 1
                a.kchan, a.n_packed = g(self.kchan), self.n_packed_d.data_ptr()
                a.tail_k, a.tail_v, a.tail_pages = g(self.tail_k), g(self.tail_v), self.tail_pages
            self._arenas[layer] = a
        return a

    def workspace(self, name: str, nbytes: int) -> torch.Tensor:
        """Zero-initialised scratch owned by the cache (grown on demand)."""
        t = self._ws.get(name)
        if t is None or t.numel() < nbytes:
            t = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=self.device)
            self._ws[name] = t
        return t

    # ------------------------------------------------------------ allocation
    def alloc_page(self, layer: int, kv_head: int, seq: int = 0) -> int:
        pid = int(self.next_page[layer, kv_head, seq])
        assert pid < self.cfg.max_pages, "KV cache is full"
        self.next_page[layer, kv_head, seq] += 1
        return pid

    def get_open_page(self, layer: int, kv_head: int, seq: int = 0) -> Optional[int]:
        n = int(self.next_page[layer, kv_head, seq])
        if n == 0:
            return None
        last = n - 1
        return last if self.valid_host[layer, kv_head, seq, last] < self.cfg.page_size else None

    def page_valid(self, layer: int, kv_head: int, page_id: int, seq: int = 0) -> int:
        return int(self.valid_host[layer, kv_head, seq, page_id])

    def num_pages(self, layer: int, kv_head: int, seq: int = 0) -> int:
        return int(self.next_page[layer, kv_head, seq])

    def all_page_ids(self, layer: int, kv_head: int, seq: int = 0) -> List[int]:
        return list(range(self.num_pages(layer, kv_head, seq)))

    def total_valid_tokens(self, layer: int, kv_head: int, seq: int = 0) -> int:
        n = self.num_pages(layer, kv_head, seq)
        return int(self.valid_host[layer, kv_head, seq, :n].sum())

    # per-page device arrays, indexed [layer, kv head, sequence, page, ...]
    _PAGE_ARRAYS = ("kcodes", "vcodes", "kscale", "vscale", "kmaster", "vmaster", "valid", "has_meta", "k_slot",
                    "v_slot", "k_err", "v_err", "k_sketch", "v_sq")

    def page_view(self, layer: int, kv_head: int, page_ids: Sequence[int], seq: int = 0) -> "CAREKVCache":
        """A one-sequence cache of the same configuration whose (layer,
        kv_head) holds pages ``page_ids`` of sequence ``seq``, in list order,
        as its pages 0..n-1, with the sequence's residual slots (slot ids
        unchanged): the page list of CAREKVAttention.forward(page_ids=...)
        (attention.py:979-990) as a prefix the decode kernels read."""
        if self.kivi_packed:
            raise NotImplementedError("page_view of a packed KIVI arena (packed prompt pages and fp16 tail)")
        pids = [int(p) for p in page_ids]
        n = len(pids)
        if n == 0 or min(pids) < 0 or max(pids) >= self.cfg.max_pages:
            raise IndexError(f"page ids must be a non-empty list in [0, {self.cfg.max_pages})")
        cfg = CacheConfig(**{**self.cfg.__dict__, "max_pages": max(n, 1)})
        v = CAREKVCache(cfg, device=self.device, n_seq=1, n_slots=self.n_slots,
                        streaming_store=self.streaming_store)
        idx = torch.tensor(pids, device=self.device)
        for nm in self._PAGE_ARRAYS:
            getattr(v, nm)[layer, kv_head, 0, :n] = getattr(self, nm)[layer, kv_head, seq].index_select(0, idx)
        for nm in ("k_res", "v_res", "k_res_scale", "v_res_scale", "next_slot"):
            getattr(v, nm)[0] = getattr(self, nm)[seq]
        v.next_page[layer, :, 0] = n  # the other kv heads' pages stay empty (no valid rows)
        v.valid_host[layer, kv_head, 0, :n] = self.valid_host[layer, kv_head, seq, pids]
        v._token_start[layer, kv_head, 0, :n] = self._token_start[layer, kv_head, seq, pids]
        return v

    def reset_sequence(self, seq: int):
        """Forget a sequence slot (pages, metadata, residual slots)."""
        self.valid[:, :, seq].zero_()
        self.has_meta[:, :, seq].zero_()
        self.k_slot[:, :, seq].fill_(-1)
        self.v_slot[:, :, seq].fill_(-1)
        self.next_slot[seq].zero_()
        self._freed.pop((seq, 0), None)
        self._freed.pop((seq, 1), None)
        self.next_page[:, :, seq] = 0
        self.valid_host[:, :, seq] = 0
        self._token_start[:, :, seq] = 0
        if self.kivi_packed:
            self.n_packed[seq] = 0
            self.n_packed_d[seq] = 0

    # ------------------------------------------------------------ page writes
    def write_prefill(self, layer: int, K: torch.Tensor, V: torch.Tensor, token_start_abs: int = 0,
                      sink_tokens: int = 4, seqs: Optional[Sequence[int]] = None):
        """Quantize + pack + store pages for a prompt chunk of every listed
        sequence (layer.py:204-334).  With a side-buffer base quantizer
        (kivi_style / kvquant_style) K_hat / V_hat are computed over the whole
        chunk first -- K per channel over T, V per token (layer.py:226-245) --
        and written as fp16 pages, the residuals taken against them.

        K, V: fp16 post-RoPE keys / values, (Hkv, T, D) for one sequence or
        (B, Hkv, T, D) with ``seqs`` naming the B sequence slots.  Returns
        (K_hat, V_hat) of the chunk for the side-buffer base, else None."""
        cfg = self.cfg
        if K.dim() == 3:
            K, V = K.unsqueeze(0), V.unsqueeze(0)
        B, H, T, D = K.shape
        assert H == cfg.num_kv_heads and D == cfg.head_dim and V.shape == K.shape
        seqs = list(range(B)) if seqs is None else list(seqs)
        assert len(seqs) == B and len(set(seqs)) == B
        if T == 0:
            return
        ps = cfg.page_size
        n_new = math.ceil(T / ps)
        pad = n_new * ps - T
        Kp, Vp = K.to(F16).contiguous(), V.to(F16).contiguous()
        hats = None
        if self.hat:
            kb, vb = hat_bits(cfg)
            Kh, Vh = kivi_qdq(Kp, kb, per_channel=True), kivi_qdq(Vp, vb, per_channel=False)
            hats = (Kh, Vh)
        pads = lambda x: torch.nn.functional.pad(x, (0, 0, 0, pad)) if pad else x  # noqa: E731
        Kp = pads(Kp).contiguous().view(B * H * n_new * ps, D)
        Vp = pads(Vp).contiguous().view(B * H * n_new * ps, D)
        Khp = Vhp = None
        if hats is not None:
            Khp = pads(hats[0]).contiguous().view(B * H * n_new * ps, D)
            Vhp = pads(hats[1]).contiguous().view(B * H * n_new * ps, D)
        kivi_in = None
        if self.kivi_packed:
            # the full pages of a prompt into empty sequences go packed, the
            # rest (a partial last page, a continuation) to the fp16 tail
            fresh = all(int(self.next_page[layer, h, s_]) == 0 for s_ in seqs for h in range(H))
            n_full = T // ps if fresh else 0
            sl = torch.tensor(seqs, device=self.device)
            if fresh:
                self.n_packed[seqs] = n_full
                self.n_packed_d[sl] = n_full
            for s_ in seqs:
                top = int(self.next_page[layer, 0, s_]) + n_new - int(self.n_packed[s_])
                if top > self.tail_pages:
                    raise _lib.CarekvError(f"packed KIVI tail full: sequence {s_} needs {top} fp16 tail pages, "
                                           f"the cache holds {self.tail_pages} (kivi_tail_pages)")
            kc, ks = kivi_codes(K.to(F16), 2, per_channel=True)    # (B, H, T, D), (B, H, D)
            vc, vs = kivi_codes(V.to(F16), 2, per_channel=False)   # (B, H, T, D), (B, H, T)
            if fresh:
                self.kchan[layer][:, sl] = ks.transpose(0, 1)
            G = D // cfg.group_size
            padc = lambda x: torch.nn.functional.pad(x, (0, 0, 0, pad)) if pad else x  # noqa: E731
            kivi_in = (padc(kc).contiguous().view(-1, D), padc(vc).contiguous().view(-1, D),
                       padc(vs.unsqueeze(-1).expand(B, H, T, G)).contiguous().view(-1, G))
        # the page jobs, sequence-major then kv head then page (the reference's
        # per-head page loop order), are generated on the device from each
        # (sequence, kv head)'s first page id: it takes the next n_new page
        # ids of its row at once
        sarr = np.asarray(seqs, dtype=np.int64)
        start = self.next_page[layer][:, sarr].T.astype(np.int64)          # (B, H)
        assert (start + n_new <= cfg.max_pages).all(), "KV cache is full"
        pr = np.arange(n_new, dtype=np.int64)
        nv = np.minimum(ps, T - pr * ps).astype(np.int32)
        tstart = (token_start_abs + pr * ps).astype(np.int32)
        for s0 in np.unique(start):  # host copies of valid / token_start, one slice per first page id
            hs, bs = np.nonzero(start.T == s0)
            self.valid_host[layer, hs, sarr[bs], s0:s0 + n_new] = nv
            self._token_start[layer, hs, sarr[bs], s0:s0 + n_new] = tstart
        self.next_page[layer][:, sarr] += n_new
        rows_d = to_device(np.concatenate([sarr, start.reshape(-1)]).astype(np.int32), self.device)
        grid = _lib.PrefillGrid(n_rows=B, n_tokens=T, token_start=int(token_start_abs), rows=rows_d.data_ptr())
        n_jobs = B * H * n_new
        knobs = resolve_store_knobs(cfg, layer)
        sp = _lib.StoreParams(k_budget=knobs.k_budget, v_budget=knobs.v_budget, joint_budget=knobs.joint_budget,
                              joint=int(knobs.joint), store_none=int(knobs.store_none),
                              sensitivity=knobs.sensitivity, sink_tokens=int(sink_tokens),
                              sketch_proj=self.sketch_proj.data_ptr(),
                              k_hat=Khp.data_ptr() if Khp is not None else None,
                              v_hat=Vhp.data_ptr() if Vhp is not None else None)
        if kivi_in is not None:
            sp.k_codes_in, sp.v_codes_in, sp.v_scale_in = (t.data_ptr() for t in kivi_in)
        lib = _lib.load()
        a = self.arena(layer)
        ws = self.workspace("store", _lib.store_workspace_bytes(lib, a, sp, n_jobs))
        ev = self.store_events  # (start, end) events around the store launches, for timing
        if ev is not None:
            ev[0].record()
        _lib.check(lib.carekv_store_prefill(a, sp, Kp.data_ptr(), Vp.data_ptr(), grid, ws.data_ptr(),
                                            _lib.stream_ptr(self.device)), "carekv_store_prefill")
        if ev is not None:
            ev[1].record()
        if _lib.check_enabled():
            _lib.check_status(ws, 4 * n_jobs, "carekv_store_prefill")
        else:
            self.status.watch(ws, 4 * n_jobs, "carekv_store_prefill")
        if self.rescale_open:  # the last page stays open: keep its rows' fp16 group scales
            last = T - (n_new - 1) * ps
            if last < ps:
                G = D // cfg.group_size
                tail = torch.cat([K[:, :, (n_new - 1) * ps:], V[:, :, (n_new - 1) * ps:]], 0).to(F16).contiguous()
                codes = torch.empty(2 * B * H * last, D, dtype=torch.int8, device=self.device)
                sc = torch.empty(2 * B * H * last, G, dtype=F16, device=self.device)
                _lib.check(lib.carekv_quantize_rows(tail.data_ptr(), 2 * B * H * last, D, cfg.base_bits, 32, 0,
                                                    codes.data_ptr(), sc.data_ptr(), _lib.stream_ptr(self.device)),
                           "carekv_quantize_rows (open page scales)")
                sc = sc.view(2, B, H, last, G)
                sl = torch.tensor(seqs, device=self.device)
                self.open_ks[layer][:, sl, :last] = sc[0].transpose(0, 1)
                self.open_vs[layer][:, sl, :last] = sc[1].transpose(0, 1)
        if self.streaming_store:  # the last page stays open: keep its true rows
            last = T - (n_new - 1) * ps
            sl = torch.tensor(seqs, device=self.device)
            self.open_k[layer, sl] = 0
            self.open_v[layer, sl] = 0
            if last < ps:
                self.open_k[layer, sl, :, :last] = K[:, :, (n_new - 1) * ps:].to(F16)
                self.open_v[layer, sl, :, :last] = V[:, :, (n_new - 1) * ps:].to(F16)
        if hats is not None:
            return hats[0] if B > 1 else hats[0][0], hats[1] if B > 1 else hats[1][0]
        return None

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor, seqs: Optional[Sequence[int]] = None):
        """Append one decode token per listed sequence and kv head
        (layer.py:1028-1146).  k, v: (Hkv, D) or (B, Hkv, D) fp16."""
        cfg = self.cfg
        if k.dim() == 2:
            k, v = k.unsqueeze(0), v.unsqueeze(0)
        B, H, D = k.shape
        seqs = list(range(B)) if seqs is None else list(seqs)
        # the row bookkeeping of every (sequence, kv head) at once: the open
        # page (the last page while it is not full) or a fresh one
        ps = cfg.page_size
        sarr = np.asarray(seqs, dtype=np.int64)
        hh, ss = np.arange(H)[None, :], sarr[:, None]
        nxt = self.next_page[layer][:, sarr].T                              # (B, H)
        vlast = self.valid_host[layer][hh, ss, np.maximum(nxt - 1, 0)]
        fresh = ~((nxt > 0) & (vlast < ps))
        if fresh.any():
            if self.kivi_packed:
                over = fresh & (nxt - self.n_packed[sarr][:, None] >= self.tail_pages)
                if over.any():
                    s_ = int(sarr[np.nonzero(over)[0][0]])
                    raise _lib.CarekvError(f"packed KIVI tail full: sequence {s_} has no fp16 tail page left "
                                           f"({self.tail_pages} per sequence, kivi_tail_pages)")
            assert (nxt[fresh] < cfg.max_pages).all(), "KV cache is full"
        pid = np.where(fresh, nxt, nxt - 1)
        if fresh.any():
            # a fresh page starts at the row's token count (pages past the row's
            # next page hold no valid rows)
            tot = self.valid_host[layer][:, sarr, :].sum(-1).T               # (B, H)
            fb, fh = np.nonzero(fresh)
            self._token_start[layer, fh, sarr[fb], pid[fb, fh]] = tot[fb, fh]
            self.next_page[layer][:, sarr] += fresh.T
        offs = self.valid_host[layer][hh, ss, pid]
        self.valid_host[layer][hh, ss, pid] = offs + 1
        dest = np.stack([np.broadcast_to(ss, (B, H)), np.broadcast_to(hh, (B, H)), pid, fresh],
                        -1).reshape(B * H, 4).astype(np.int32)
        fb, fh = np.nonzero(offs + 1 == ps)
        filled = [(int(sarr[b_]), int(h_), int(pid[b_, h_])) for b_, h_ in zip(fb, fh)]  # the pages the appends fill
        offs = offs.reshape(B * H).astype(np.int64)
        # one upload: the page destinations (int32 [B*H][4]) and, with the
        # streaming store, the rows of the open-page buffers (seq, head, offset)
        # flattened (int64 [B*H])
        n = B * H
        buf = np.empty(2 * n + (n if self.streaming_store else 0), dtype=np.int64)
        buf[:2 * n].view(np.int32)[:] = dest.reshape(-1)
        if self.streaming_store:
            buf[2 * n:] = (dest[:, 0].astype(np.int64) * H + dest[:, 1]) * ps + offs
        buf_d = to_device(buf, self.device)
        dest_d = buf_d[:2 * n].view(torch.int32)
        kk = k.to(F16).contiguous().view(B * H, D)
        vv = v.to(F16).contiguous().view(B * H, D)
        lib = _lib.load()
        _lib.check(lib.carekv_append_rows(self.arena(layer), kk.data_ptr(), vv.data_ptr(), dest_d.data_ptr(), B * H,
                                          _lib.stream_ptr(self.device)), "carekv_append_rows")
        if self.streaming_store:
            rows = buf_d[2 * n:]
            self.open_k[layer].view(-1, D).index_copy_(0, rows, kk)
            self.open_v[layer].view(-1, D).index_copy_(0, rows, vv)
            if filled:
                self._streaming_fill_store(layer, filled)

    def _streaming_fill_store(self, layer: int, filled):
        """Store the filled pages' residuals from their true rows against the
        pages' own base (carekv_store_pages with keep_base), as the fill store
        of layer.py:1128-1146 with K_orig = the true rows."""
        cfg = self.cfg
        ps = cfg.page_size
        filled = sorted(filled)  # grouped by sequence, kv heads in order
        jobs = np.zeros((len(filled), _lib.PAGE_JOB_INTS), dtype=np.int32)
        seqs = sorted({f[0] for f in filled})
        group_ptr = np.zeros(len(seqs) + 1, dtype=np.int32)
        for j, (s, h, pid) in enumerate(filled):
            jobs[j] = (s, h, pid, ps, int(self._token_start[layer, h, s, pid]), 1)
            group_ptr[seqs.index(s) + 1] = j + 1
        idx = to_device(np.array(filled, dtype=np.int64).T.copy(), self.device)  # (seq, head, page) rows
        si, hi = idx[0], idx[1]
        Kp = self.open_k[layer, si, hi].contiguous().view(-1, cfg.head_dim)
        Vp = self.open_v[layer, si, hi].contiguous().view(-1, cfg.head_dim)
        knobs = resolve_store_knobs(cfg, layer)
        sp = _lib.StoreParams(k_budget=knobs.k_budget, v_budget=knobs.v_budget, joint_budget=knobs.joint_budget,
                              joint=int(knobs.joint), store_none=int(knobs.store_none),
                              sensitivity=knobs.sensitivity, sink_tokens=4,
                              sketch_proj=self.sketch_proj.data_ptr(), keep_base=0 if self.hat else 1,
                              reuse_slots=1)
        keep = []
        if self.hat:  # the fp16 base: the pages' own K_hat / V_hat rows as the residual base
            pi = idx[2]
            if self.kivi_packed:  # filled pages are tail pages
                ti = pi - to_device(self.n_packed.astype(np.int64), self.device)[si]
                Khat = self.tail_k[layer, hi, si, ti].contiguous().view(-1, cfg.head_dim)
                Vhat = self.tail_v[layer, hi, si, ti].contiguous().view(-1, cfg.head_dim)
                zc = torch.zeros(Khat.shape, dtype=torch.int8, device=self.device)
                zs = torch.zeros(Khat.shape[0], cfg.head_dim // cfg.group_size, dtype=F16, device=self.device)
                keep += [zc, zs]
                sp.k_codes_in, sp.v_codes_in, sp.v_scale_in = zc.data_ptr(), zc.data_ptr(), zs.data_ptr()
            else:
                Khat = self.kcodes[layer, hi, si, pi].view(F16).contiguous().view(-1, cfg.head_dim)
                Vhat = self.vcodes[layer, hi, si, pi].view(F16).contiguous().view(-1, cfg.head_dim)
            sp.k_hat, sp.v_hat = Khat.data_ptr(), Vhat.data_ptr()
        lib = _lib.load()
        ws = self.workspace("store", _lib.store_workspace_bytes(lib, self.arena(layer), sp, len(jobs)))
        jobs_d = to_device(jobs, self.device)
        gp_d = to_device(group_ptr, self.device)
        _lib.check(lib.carekv_store_pages(self.arena(layer), sp, Kp.data_ptr(), Vp.data_ptr(), jobs_d.data_ptr(),
                                          len(jobs), gp_d.data_ptr(), len(seqs), ws.data_ptr(),
                                          _lib.stream_ptr(self.device)), "carekv_store_pages (streaming)")
        if _lib.check_enabled():
            _lib.check_status(ws, 4 * len(jobs), "carekv_store_pages (streaming)")
        else:
            self.status.watch(ws, 4 * len(jobs), "carekv_store_pages (streaming)")
        self.open_k[layer, si, hi] = 0
        self.open_v[layer, si, hi] = 0

    # ------------------------------------------------------------ reads
    def read_base_hat_concat(self, layer: int, kv_head: int, page_ids: Optional[List[int]] = None, seq: int = 0):
        """(K_hat fp16 (N, D), V_hat fp16 (N, D), valid_lens) of the fp16
        side buffer (cache.py:841-865)."""
        if not self.hat:
            raise _lib.CarekvError("read_base_hat_concat needs a side-buffer base quantizer")
        n = self.num_pages(layer, kv_head, seq)
        pids = list(range(n)) if page_ids is None else list(page_ids)
        lens = [int(self.valid_host[layer, kv_head, seq, p]) for p in pids]
        D = self.cfg.head_dim
        if self.kivi_packed:  # packed prompt pages dequantised, tail pages copied (carekv_read_hat_pages)
            N = sum(lens)
            kh = torch.zeros(N, D, dtype=F16, device=self.device)
            vh = torch.zeros_like(kh)
            if N:
                rs = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)).to(self.device)
                pl = torch.tensor(pids, dtype=torch.int32, device=self.device)
                lib = _lib.load()
                _lib.check(lib.carekv_read_hat_pages(self.arena(layer), seq, kv_head, len(pids), pl.data_ptr(),
                                                     rs.data_ptr(), kh.data_ptr(), vh.data_ptr(),
                                                     _lib.stream_ptr(self.device)), "carekv_read_hat_pages")
            return kh, vh, lens
        kh = self.kcodes[layer, kv_head, seq].view(F16).view(self.cfg.max_pages, self.cfg.page_size, D)
        vh = self.vcodes[layer, kv_head, seq].view(F16).view(self.cfg.max_pages, self.cfg.page_size, D)
        ks = [kh[p, :n_] for p, n_ in zip(pids, lens) if n_]
        vs = [vh[p, :n_] for p, n_ in zip(pids, lens) if n_]
        if not ks:
            e = torch.zeros(0, D, dtype=F16, device=self.device)
            return e, e, lens
        return torch.cat(ks), torch.cat(vs), lens

    def read_base_concat(self, layer: int, kv_head: int, page_ids: Optional[List[int]] = None, seq: int = 0):
        """(K_codes int8 (N, D), K_scale fp16 (N, G), V_codes, V_scale, valid_lens)
        for the valid rows of the listed pages (all pages when None), in list
        order (cache.py:720-772)."""
        n_all = self.num_pages(layer, kv_head, seq)
        pids = list(range(n_all)) if page_ids is None else [int(p) for p in page_ids]
        if any(p < 0 or p >= self.cfg.max_pages for p in pids):
            raise IndexError(f"page ids must lie in [0, {self.cfg.max_pages})")
        if self.hat:
            raise _lib.CarekvError("read_base_concat needs a packed base (use read_base_hat_concat)")
        lens = [int(self.valid_host[layer, kv_head, seq, p]) for p in pids]
        N = sum(lens)
        D, G = self.cfg.head_dim, self.cfg.head_dim // self.cfg.group_size
        kc = torch.zeros(N, D, dtype=torch.int8, device=self.device)
        vc = torch.zeros_like(kc)
        ks = torch.zeros(N, G, dtype=F16, device=self.device)
        vs = torch.zeros_like(ks)
        if N:
            rs = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)).to(self.device)
            pl = torch.tensor(pids, dtype=torch.int32, device=self.device)
            lib = _lib.load()
            _lib.check(lib.carekv_read_pages(self.arena(layer), seq, kv_head, len(pids), pl.data_ptr(), rs.data_ptr(),
                                             kc.data_ptr(), ks.data_ptr(), vc.data_ptr(), vs.data_ptr(),
                                             _lib.stream_ptr(self.device)), "carekv_read_pages")
            torch.cuda.current_stream(self.device).synchronize()
        return kc, ks, vc, vs, lens

    def read_base(self, layer: int, kv_head: int, page_ids: List[int], seq: int = 0):
        """cache.py:776-798: every row (padding included) of the listed pages,
        (K_codes (P*T, D) int8, K_scale (P*T, G) fp16, V_codes, V_scale)."""
        from .quantizer import unpack_codes_2d
        if self.hat:
            raise _lib.CarekvError("read_base needs a packed base")
        cfg = self.cfg
        pl = torch.tensor([int(p) for p in page_ids], dtype=torch.long, device=self.device)
        out = []
        for codes, sc, master in ((self.kcodes, self.kscale, self.kmaster), (self.vcodes, self.vscale, self.vmaster)):
            rows = codes[layer, kv_head, seq, pl].reshape(-1, self._packed_row_bytes)
            c = unpack_codes_2d(rows, cfg.base_bits, cfg.head_dim)
            s_ = sc[layer, kv_head, seq, pl]
            if self.scale_mode:  # cache.py:713-718: half(code * master)
                s_ = (s_.float() * master[layer, kv_head, seq, pl].float()[:, None, None]).to(F16)
            out += [c, s_.reshape(-1, s_.shape[-1])]
        return out[0], out[1], out[2], out[3]

    # ------------------------------------------------------------ reference page / slot interface
    def alloc_k_slot(self, seq: int = 0) -> int:
        """cache.py:548-557: the next free K slot id of the sequence (ascending,
        then the freed ones in the order they were freed).  The store kernels
        allocate from the same counter; they do not reuse freed ids."""
        return self._alloc_slot(seq, 0)

    def alloc_v_slot(self, seq: int = 0) -> int:
        """cache.py:559-561."""
        return self._alloc_slot(seq, 1)

    def free_k_slot(self, slot: int, seq: int = 0):
        """cache.py:563-564."""
        self._freed.setdefault((seq, 0), []).append(int(slot))

    def free_v_slot(self, slot: int, seq: int = 0):
        """cache.py:566-567."""
        self._freed.setdefault((seq, 1), []).append(int(slot))

    def _alloc_slot(self, seq: int, kind: int) -> int:
        nxt = int(self.next_slot[seq, kind].item())
        if nxt < self.n_slots:
            self.next_slot[seq, kind] = nxt + 1
            return nxt
        freed = self._freed.get((seq, kind), [])
        assert freed, ("K" if kind == 0 else "V") + " residual buffer is full"
        return freed.pop(0)

    def write_base(self, layer: int, kv_head: int, page_id: int, K_codes: torch.Tensor, K_scale: torch.Tensor,
                   V_codes: torch.Tensor, V_scale: torch.Tensor, num_valid: int, seq: int = 0):
        """cache.py:617-654 through carekv_write_base: pack the page's codes
        ((T, D) int8, zero padded to the page), encode its (T, G) fp16 scales
        (int8 codes under a per-page master with scale_quant=int8), record
        num_valid."""
        cfg = self.cfg
        assert 0 <= num_valid <= cfg.page_size, num_valid
        if self.hat:
            raise _lib.CarekvError("write_base needs a packed base (use write_base_kivi)")
        pad = lambda t: torch.nn.functional.pad(t, (0, 0, 0, cfg.page_size - t.shape[0])) if t.shape[0] < cfg.page_size else t  # noqa: E731,E501
        kc, vc = pad(K_codes.to(torch.int8)).contiguous(), pad(V_codes.to(torch.int8)).contiguous()
        ksc, vsc = pad(K_scale.to(F16)).contiguous(), pad(V_scale.to(F16)).contiguous()
        for t in (kc, vc, ksc, vsc):
            _lib.ptr(t)
        lib = _lib.load()
        _lib.check(lib.carekv_write_base(self.arena(layer), seq, kv_head, page_id, kc.data_ptr(), ksc.data_ptr(),
                                         vc.data_ptr(), vsc.data_ptr(), int(num_valid),
                                         _lib.stream_ptr(self.device)), "carekv_write_base")
        self.valid_host[layer, kv_head, seq, page_id] = num_valid
        if self.rescale_open and num_valid < cfg.page_size:  # the open page's fp16 scales, for the re-encoding append
            self.open_ks[layer, kv_head, seq, :num_valid] = ksc[:num_valid]
            self.open_vs[layer, kv_head, seq, :num_valid] = vsc[:num_valid]

    def append_to_page(self, layer: int, kv_head: int, page_id: int, K_codes_row: torch.Tensor,
                       K_scale_row: torch.Tensor, V_codes_row: torch.Tensor, V_scale_row: torch.Tensor,
                       seq: int = 0) -> int:
        """cache.py:656-701: append one quantized row ((D,) int8 codes, (G,)
        fp16 scales) at the page's next offset; returns the offset.  The int8
        scale encoding is the cache's (the reference's fixed master under
        cfg.compat, else the page re-encoded as write_base encodes it)."""
        cfg = self.cfg
        off = int(self.valid_host[layer, kv_head, seq, page_id])
        assert off < cfg.page_size, "page already full"
        dest = torch.tensor([[seq, kv_head, page_id, int(off == 0)]], dtype=torch.int32, device=self.device)
        kc = K_codes_row.to(torch.int8).reshape(1, -1).contiguous()
        vc = V_codes_row.to(torch.int8).reshape(1, -1).contiguous()
        ksc = K_scale_row.to(F16).reshape(1, -1).contiguous()
        vsc = V_scale_row.to(F16).reshape(1, -1).contiguous()
        for t in (kc, vc, ksc, vsc):
            _lib.ptr(t)
        lib = _lib.load()
        _lib.check(lib.carekv_append_coded_rows(self.arena(layer), kc.data_ptr(), ksc.data_ptr(), vc.data_ptr(),
                                                vsc.data_ptr(), dest.data_ptr(), 1, _lib.stream_ptr(self.device)),
                   "carekv_append_coded_rows")
        self.valid_host[layer, kv_head, seq, page_id] = off + 1
        return off

    def write_base_kivi(self, layer: int, kv_head: int, page_id: int, K_hat: torch.Tensor, V_hat: torch.Tensor,
                        num_valid: int, seq: int = 0):
        """cache.py:800-818: the page's fp16 K_hat / V_hat rows (side buffer)."""
        assert self.hat, "write_base_kivi requires a side-buffer base quantizer"
        assert 0 <= num_valid <= self.cfg.page_size, num_valid
        T = K_hat.shape[0]
        kp, vp = self._hat_page(layer, kv_head, page_id, seq)
        kp[:T] = K_hat.to(F16)
        vp[:T] = V_hat.to(F16)
        self.valid[layer, kv_head, seq, page_id] = num_valid
        self.valid_host[layer, kv_head, seq, page_id] = num_valid

    def append_to_page_kivi(self, layer: int, kv_head: int, page_id: int, K_hat_row: torch.Tensor,
                            V_hat_row: torch.Tensor, seq: int = 0) -> int:
        """cache.py:820-838: one fp16 K_hat / V_hat row at the page's next offset."""
        assert self.hat, "append_to_page_kivi requires a side-buffer base quantizer"
        off = int(self.valid_host[layer, kv_head, seq, page_id])
        assert off < self.cfg.page_size, "page already full"
        kp, vp = self._hat_page(layer, kv_head, page_id, seq)
        kp[off] = K_hat_row.to(F16)
        vp[off] = V_hat_row.to(F16)
        self.valid[layer, kv_head, seq, page_id] = off + 1
        self.valid_host[layer, kv_head, seq, page_id] = off + 1
        return off

    def _hat_page(self, layer: int, kv_head: int, page_id: int, seq: int):
        """(K_hat, V_hat) fp16 (page_size, D) views of a side-buffer page; on
        a packed KIVI cache only the fp16 tail pages have them."""
        if self.kivi_packed:
            tp = page_id - int(self.n_packed[seq])
            if not 0 <= tp < self.tail_pages:
                raise _lib.CarekvError(f"page {page_id} of a packed KIVI cache is not an fp16 tail page "
                                       f"(packed pages: {int(self.n_packed[seq])}, tail pages: {self.tail_pages})")
            return self.tail_k[layer, kv_head, seq, tp], self.tail_v[layer, kv_head, seq, tp]
        return (self.kcodes[layer, kv_head, seq, page_id].view(F16), self.vcodes[layer, kv_head, seq, page_id].view(F16))

    def write_k_residual(self, slot: int, packed: torch.Tensor, scale: torch.Tensor, seq: int = 0):
        """cache.py:871-873."""
        self.k_res[seq, slot] = packed.flatten().to(torch.int8)
        self.k_res_scale[seq, slot] = scale.flatten()[0].to(F16)

    def write_v_residual(self, slot: int, packed: torch.Tensor, scale: torch.Tensor, seq: int = 0):
        """cache.py:875-877."""
        self.v_res[seq, slot] = packed.flatten().to(torch.int8)
        self.v_res_scale[seq, slot] = scale.flatten()[0].to(F16)

    def read_k_residual(self, slot: int, seq: int = 0):
        """cache.py:879-880: (packed (slot_bytes,) int8, scale (1,) fp16)."""
        return self.k_res[seq, slot], self.k_res_scale[seq, slot:slot + 1]

    def read_v_residual(self, slot: int, seq: int = 0):
        """cache.py:882-883."""
        return self.v_res[seq, slot], self.v_res_scale[seq, slot:slot + 1]

    def page_meta(self, layer: int, kv_head: int, page_id: int, seq: int = 0) -> Optional[PageMeta]:
        idx = (layer, kv_head, seq, page_id)
        if not int(self.has_meta[idx].item()):
            return None
        return PageMeta(page_id=page_id, layer_id=layer, kv_head=kv_head,
                        token_start=int(self._token_start[idx]), num_tokens=int(self.valid_host[idx]),
                        k_residual_slots=self.k_slot[idx].tolist(), v_residual_slots=self.v_slot[idx].tolist(),
                        k_error_norm=self.k_err[idx].clone(), v_error_norm=self.v_err[idx].clone(),
                        k_sketch=self.k_sketch[idx].clone())

    @property
    def meta_table(self):
        """[layer][kv_head][page] -> PageMeta | None for sequence 0 (reads the device)."""
        cfg = self.cfg
        return [[[self.page_meta(l, h, p) for p in range(cfg.max_pages)] for h in range(cfg.num_kv_heads)]
                for l in range(cfg.num_layers)]

    def num_stored_residual_slots(self, seq: int = 0) -> Tuple[int, int]:
        ns = self.next_slot[seq].tolist()
        return int(ns[0]), int(ns[1])

    # reference-shaped views for a single-sequence cache
    def _view(self, t):
        return t[:, :, 0] if self.n_seq == 1 else t

    base_K_hat_fp16 = property(lambda self: self._view(self.kcodes).view(F16)
                               if self.hat and not self.kivi_packed else None)
    base_V_hat_fp16 = property(lambda self: self._view(self.vcodes).view(F16)
                               if self.hat and not self.kivi_packed else None)
    base_K_codes = property(lambda self: self._view(self.kcodes))
    base_V_codes = property(lambda self: self._view(self.vcodes))
    base_K_scale = property(lambda self: self._view(self.kscale))
    base_V_scale = property(lambda self: self._view(self.vscale))
    base_K_scale_master = property(lambda self: self._view(self.kmaster) if self.scale_mode else None)
    base_V_scale_master = property(lambda self: self._view(self.vmaster) if self.scale_mode else None)
    valid_tokens = property(lambda self: self._view(self.valid))
    k_residual_buf = property(lambda self: self.k_res[0] if self.n_seq == 1 else self.k_res)
    v_residual_buf = property(lambda self: self.v_res[0] if self.n_seq == 1 else self.v_res)
    k_residual_scale = property(lambda self: (self.k_res_scale[0] if self.n_seq == 1 else self.k_res_scale).unsqueeze(-1))
    v_residual_scale = property(lambda self: (self.v_res_scale[0] if self.n_seq == 1 else self.v_res_scale).unsqueeze(-1))
