"""``CAREKVLayer``: the per-layer prefill / decode driver (layer.py:147-1163 of
the reference), batched over sequences, with every CARE-KV computation in
the HIP library:

* projections and RoPE stay torch matmuls / elementwise ops on the caller's
  device (the reference does the same, layer.py:665-690, 996-1014);
* the page store (quantize, pack, residual candidates, slots) is
  ``CAREKVCache.write_prefill`` (``carekv_store_pages``);
* the decode append with store-on-fill is ``CAREKVCache.append``
  (``carekv_append_rows``);
* prefill attention is ``prefill_attention`` over (K_post, V) in the ``fp``
  mode or over the fp16-scale K_hat / V_hat in the quantised modes
  (``carekv_prefill_attn``, layer.py:759-781), plus the stored-slot sparse
  correction in ``carekv_stored`` mode (``prefill_correction``,
  ``carekv_prefill_correct``, layer.py:808-838) or the in-memory one in
  ``carekv_eval`` mode (``prefill_eval``, ``carekv_prefill_eval``,
  layer.py:363-456, 792-806);
* decode attention with the comb+ex correction is ``decode_attention``
  (``carekv_decode_attn``, layer.py:1148-1160).
"""
from __future__ import annotations

import os
from typing import Any, Dict, Optional, Sequence, Tuple

import torch
from torch import Tensor, nn

from .attention import (debug_stats_enabled, decode_attention, decode_read_mode, get_debug_stats,  # noqa: F401
                        get_imp_per_layer, importance_probe, prefill_correction, reset_debug_stats)
from .cache import CAREKVCache
from .config import CacheConfig, any_read_budget, resolve_read_knobs
from .prefill import eval_knobs, prefill_attention, prefill_eval, quant_dequant

try:  # the reference takes RoPE from transformers as well (layer.py:65-69)
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
except Exception:  # pragma: no cover - transformers missing
    apply_rotary_pos_emb = None

F16 = torch.float16
PREFILL_MODES = ("fp", "base_quant", "carekv_eval", "carekv_stored")


def resolve_prefill_mode() -> str:
    """``_resolve_prefill_mode`` (layer.py:129-140)."""
    raw = os.environ.get("CAREKV_PREFILL_MODE", "fp").lower()
    if raw == "carekv":
        return "carekv_eval"
    if raw in {"quant", "int"}:
        return "base_quant"
    if raw not in PREFILL_MODES:
        raise ValueError(f"CAREKV_PREFILL_MODE={raw!r} is not one of {PREFILL_MODES}")
    return raw


def prefill_read_knobs(cfg: CacheConfig, layer_id: int):
    """Read knobs of the carekv_stored prefill correction by
    cfg.correction_impl (layer.py:514-557): ``vectorized`` runs
    vectorized_joint_correction, whose K score follows CAREKV_KSCORE_LIVE;
    ``cached`` / ``python`` run apply_slot_corrections per (head, row) over
    ResidualRouter.route, which has no query-aware K score (the sketch
    proxy, whatever CAREKV_KSCORE_LIVE says)."""
    knobs = resolve_read_knobs(cfg, layer_id)
    if cfg.correction_impl != "vectorized":
        knobs.kscore_live = False
    return knobs


def _rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> Tuple[Tensor, Tensor]:
    """q (B, Hq, T, D), k (B, Hkv, T, D); cos/sin (B or 1, T, rot)."""
    if apply_rotary_pos_emb is not None:
        return apply_rotary_pos_emb(q, k, cos, sin)
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)

    def rot(x):
        h = x.shape[-1] // 2
        return torch.cat((-x[..., h:], x[..., :h]), dim=-1)
    return q * c + rot(q) * s, k * c + rot(k) * s


class CAREKVLayer(nn.Module):
    """Drop-in attention layer over the CARE-KV cache (layer.py:147-183)."""

    def __init__(self, cfg: CacheConfig, layer_id: int, W_Q: Tensor, W_K: Tensor, W_V: Tensor, W_O: Tensor,
                 device: Optional[torch.device] = None):
        super().__init__()
        self.cfg = cfg
        self.layer_id = layer_id
        self.device = torch.device(device) if device is not None else W_Q.device
        self.W_Q = nn.Parameter(W_Q, requires_grad=False)
        self.W_K = nn.Parameter(W_K, requires_grad=False)
        self.W_V = nn.Parameter(W_V, requires_grad=False)
        self.W_O = nn.Parameter(W_O, requires_grad=False)

    # ------------------------------------------------------------ helpers
    def _project(self, hidden: Tensor):
        """hidden (B, T, model_dim) -> Q (B, Hq, T, D), K/V (B, Hkv, T, D)."""
        cfg = self.cfg
        B, T, _ = hidden.shape
        Hq, Hkv, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        Q = (hidden @ self.W_Q.T).reshape(B, T, Hq, D).transpose(1, 2)
        K = (hidden @ self.W_K.T).reshape(B, T, Hkv, D).transpose(1, 2)
        V = (hidden @ self.W_V.T).reshape(B, T, Hkv, D).transpose(1, 2)
        return Q, K, V

    def _out(self, O: Tensor, dtype) -> Tensor:
        """O (B, Hq, T, D) -> (B, T, model_dim) through W_O."""
        B, Hq, T, D = O.shape
        return O.transpose(1, 2).reshape(B, T, Hq * D).to(self.W_O.dtype) @ self.W_O.T

    @staticmethod
    def _key_runs(attention_mask: Optional[Tensor], B: int, T: int) -> Optional[list]:
        """Each sequence's run of real tokens [s, e) of the T prompt rows, or
        None when every sequence sees all of them (the kernel applies the
        causal mask itself, as the attention_mask=None branch of
        layer.py:951-962 does).

        The mask is the one layer.py:952-957 adds to the scores: (T, T),
        (B or 1, T, T) or (B or 1, 1, T, T), boolean (True: visible) or
        additive (0: visible, at most half the dtype's lowest value:
        masked); a (B, S) keep-mask (nonzero: a real token) is read as
        HF's models take it.  A sequence's real tokens are the keys its last
        query row sees; they must form one run (left or right padding).
        Other additive values (a bias the kernel would not apply) and
        visible sets with holes are refused."""
        if attention_mask is None or not torch.is_tensor(attention_mask):
            return None
        m = attention_mask
        if m.dim() == 2 and tuple(m.shape) != (T, T) and m.shape[0] == B and m.shape[1] >= T:
            vis = m[:, -T:] != 0                       # (B, S) keep-mask
        else:
            if m.dim() == 4:
                m = m[:, 0]
            if m.dim() == 2:
                m = m.unsqueeze(0)
            if m.dim() != 3 or m.shape[-1] < T or m.shape[-2] < T:
                raise NotImplementedError(f"attention mask of shape {tuple(attention_mask.shape)}: expected "
                                          "(T, T), (B, T, T), (B, 1, T, T) or a (B, S) keep-mask")
            m = m[:, -T:, -T:]
            if m.dtype == torch.bool:
                vis = m[:, -1]
            else:
                lo = torch.finfo(m.dtype).min / 2 if m.dtype.is_floating_point else -1
                if bool((~((m == 0) | (m <= lo))).any()):
                    raise NotImplementedError("an additive attention mask with values other than 0 and the "
                                              "masked minimum (a score bias) is not applied by the prefill kernel")
                vis = m[:, -1] == 0
        if bool(vis.all()):
            return None
        if vis.shape[0] not in (1, B):
            raise NotImplementedError(f"attention mask batch {vis.shape[0]} for {B} sequences")
        vis = vis.expand(B, T).cpu()
        runs = []
        for b in range(B):
            idx = torch.nonzero(vis[b]).flatten()
            s, e = (int(idx[0]), int(idx[-1]) + 1) if idx.numel() else (0, 0)
            if e - s != idx.numel():
                raise NotImplementedError(f"sequence {b}: the visible keys of its last row are not one run "
                                          "(only left or right padding is supported)")
            runs.append((s, e))
        return runs

    def _prefill_runs(self, cache: CAREKVCache, hidden: Tensor, runs, sink_tokens: int,
                      position_embeddings, token_start_abs: int, seqs: Sequence[int]) -> Tensor:
        """A padded batch: the sequences whose rows are all real run as one
        batch, every other sequence alone over its real rows [s, e) (RoPE
        rows sliced alike), so no pad row reaches a page or an attention
        row.  Pad rows of the output are zero."""
        B, T, _ = hidden.shape
        out = hidden.new_zeros((B, T, self.W_O.shape[0]))

        def pe(rows, sl):
            if position_embeddings is None:
                return None
            return tuple((x[rows] if x.shape[0] == B else x[[0] * len(rows)])[:, sl] for x in position_embeddings)
        full = [b for b, (s, e) in enumerate(runs) if (s, e) == (0, T)]
        if full:
            out[full] = self.prefill(cache, hidden[full], sink_tokens=sink_tokens,
                                     position_embeddings=pe(full, slice(None)), token_start_abs=token_start_abs,
                                     seqs=[seqs[b] for b in full])
        for b, (s, e) in enumerate(runs):
            if (s, e) != (0, T) and e > s:
                out[b, s:e] = self.prefill(cache, hidden[b:b + 1, s:e], sink_tokens=sink_tokens,
                                           position_embeddings=pe([b], slice(s, e)),
                                           token_start_abs=token_start_abs, seqs=[seqs[b]])[0]
        return out

    # ------------------------------------------------------------ prefill
    def prefill(self, cache: CAREKVCache, hidden: Tensor, sink_tokens: int = 4,
                attention_mask: Optional[Tensor] = None,
                position_embeddings: Optional[Tuple[Tensor, Tensor]] = None, token_start_abs: int = 0,
                debug_stats: Optional[Dict[str, Any]] = None, seqs: Optional[Sequence[int]] = None) -> Tensor:
        """layer.py:643-935 for a batch: hidden (T, model_dim) or (B, T,
        model_dim) -> the attention output through W_O, same leading shape.

        Every mode writes the pages (post-RoPE K, layer.py:719-737).  The
        output is attention over (K_post, V) in ``fp`` mode and over the
        dequantised K_hat / V_hat otherwise; ``carekv_stored`` adds the
        sparse correction from the stored slots (``prefill_correction``,
        layer.py:808-838), ``carekv_eval`` the token-level correction from
        the full in-memory residuals (``prefill_eval``, layer.py:363-456).

        A padding mask (left or right padding) keeps each sequence's pad
        rows out of its pages and its attention: those sequences run over
        their real rows alone and their pad rows return zero.  The reference
        adds the mask to one sequence's scores and still stores the pad rows
        (layer.py:952-957); its B > 1 loop cannot broadcast a batched mask."""
        squeeze = hidden.dim() == 2
        if squeeze:
            hidden = hidden.unsqueeze(0)
        cfg = self.cfg
        B, T, _ = hidden.shape
        mode = resolve_prefill_mode()
        seqs = list(range(B)) if seqs is None else list(seqs)
        runs = self._key_runs(attention_mask, B, T)
        if runs is not None:
            out = self._prefill_runs(cache, hidden, runs, sink_tokens, position_embeddings, token_start_abs, seqs)
            return out[0] if squeeze else out
        Q, K, V = self._project(hidden)
        if position_embeddings is not None:
            cos, sin = position_embeddings
            Q, K = _rope(Q, K, cos.to(Q.dtype), sin.to(Q.dtype))
        Qh, Kh, Vh = Q.to(F16).contiguous(), K.to(F16).contiguous(), V.to(F16).contiguous()
        hats = cache.write_prefill(self.layer_id, Kh, Vh, token_start_abs=token_start_abs,
                                   sink_tokens=sink_tokens, seqs=seqs)
        if mode == "fp":
            O = prefill_attention(Qh, Kh, Vh)
        else:
            if hats is not None:  # side-buffer base: the K_hat / V_hat the pages hold (layer.py:328-332)
                Khat, Vhat = (hats[0].unsqueeze(0), hats[1].unsqueeze(0)) if hats[0].dim() == 3 else hats
            else:
                Khat = quant_dequant(Kh, cfg.base_bits, cfg.group_size)
                Vhat = quant_dequant(Vh, cfg.base_bits, cfg.group_size)
            stored = mode == "carekv_stored" and any_read_budget(cfg)
            if stored and token_start_abs != 0:
                raise NotImplementedError("carekv_stored prefill correction of a prompt continuation "
                                          "(token_start_abs > 0): the reference scores one prompt at a time")
            # the stored-slot correction weighs the prompt rows with the base's
            # log-sum-exp; the other modes need only O
            O, lse = prefill_attention(Qh, Khat, Vhat, return_lse=True) if stored else \
                (prefill_attention(Qh, Khat, Vhat), None)
            if mode == "carekv_eval":  # layer.py:792-806: full in-memory residuals
                O = prefill_eval(Qh, Kh, Vh, Khat, Vhat, O, **eval_knobs(cfg.read_budget_ratio))
            if stored:  # layer.py:808-838: the sparse correction from the stored slots
                knobs = prefill_read_knobs(cfg, self.layer_id)
                if os.environ.get("CAREKV_DUMP_IMPORTANCE", "0") == "1" and debug_stats_enabled():
                    for b in range(len(seqs)):  # layer.py:477-502
                        importance_probe(self.layer_id, Qh[b], Khat[b])
                for b, sq in enumerate(seqs):
                    O[b] = prefill_correction(cache, self.layer_id, Qh[b].transpose(0, 1), Khat[b], Vhat[b],
                                              lse[b], seq=sq, knobs=knobs).transpose(0, 1)
        out = self._out(O, hidden.dtype).to(hidden.dtype)
        return out[0] if squeeze else out

    # ------------------------------------------------------------ decode
    def decode_step(self, cache: CAREKVCache, hidden: Tensor,
                    position_embeddings: Optional[Tuple[Tensor, Tensor]] = None,
                    debug_stats: Optional[Dict[str, Any]] = None, seqs: Optional[Sequence[int]] = None) -> Tensor:
        """layer.py:978-1163 for a batch: hidden (1, model_dim) of one
        sequence or (B, 1, model_dim) -> same shape.  Appends the token's
        K / V (store on page fill with K_orig = K_hat, layer.py:1088-1146),
        then runs the decode attention with the correction
        ``decode_read_mode`` resolves."""
        squeeze = hidden.dim() == 2
        if squeeze:
            hidden = hidden.unsqueeze(0)
        B = hidden.shape[0]
        Q, K, V = self._project(hidden[:, -1:])
        if position_embeddings is not None:
            cos, sin = position_embeddings
            Q, K = _rope(Q, K, cos.to(Q.dtype), sin.to(Q.dtype))
        seqs = list(range(B)) if seqs is None else list(seqs)
        cache.append(self.layer_id, K[:, :, 0].to(F16), V[:, :, 0].to(F16), seqs=seqs)
        correction, knobs = decode_read_mode(self.cfg, self.layer_id)
        O = decode_attention(cache, self.layer_id, Q[:, :, 0].to(F16), seqs=seqs, correction=correction,
                             knobs=knobs)  # (B, Hq, D)
        out = self._out(O.unsqueeze(2), hidden.dtype).to(hidden.dtype)  # (B, 1, model_dim)
        return out[0] if squeeze else out
