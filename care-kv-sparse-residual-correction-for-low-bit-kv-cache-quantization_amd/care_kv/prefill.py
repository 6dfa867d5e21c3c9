"""Prefill-side operators: exact quantize / dequantize of rows, the causal
attention over dequantised K/V (``CAREKVLayer._causal_attention_pure``,
layer.py:935-972) and the in-memory ``carekv_eval`` correction
(``_apply_sparse_prefill_correction_eval``, layer.py:363-456), all on the HIP
library."""
from __future__ import annotations

import math
import os
from typing import Optional, Tuple

import torch

from . import _lib


def quantize_rows(x: torch.Tensor, bits: int, group: int = 32, pack: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """``quantize`` (quantizer.py:31-64) in fp16 arithmetic over the last dim.

    x: (..., D) fp16 -> codes int8 (..., D) (or packed (..., D*bits/8) with
    ``pack``) and fp16 group scales (..., D/group)."""
    x = x.to(torch.float16).contiguous()
    D = x.shape[-1]
    rows = x.numel() // D
    lead = x.shape[:-1]
    nb = D * bits // 8 if pack else D
    codes = torch.empty(*lead, nb, dtype=torch.int8, device=x.device)
    scale = torch.empty(*lead, D // group, dtype=torch.float16, device=x.device)
    lib = _lib.load()
    _lib.check(lib.carekv_quantize_rows(_lib.ptr(x), rows, D, bits, group, int(bool(pack)), _lib.ptr(codes),
                                        _lib.ptr(scale), _lib.stream_ptr(x.device)), "carekv_quantize_rows")
    return codes, scale


def dequantize_rows(codes: torch.Tensor, scale: torch.Tensor, group: int = 32) -> torch.Tensor:
    """``dequantize`` (quantizer.py:67-82): half(code * scale), unpacked codes."""
    codes = codes.contiguous()
    scale = scale.to(torch.float16).contiguous()
    D = codes.shape[-1]
    rows = codes.numel() // D
    out = torch.empty(codes.shape, dtype=torch.float16, device=codes.device)
    lib = _lib.load()
    _lib.check(lib.carekv_dequantize_rows(_lib.ptr(codes), _lib.ptr(scale), rows, D, group, _lib.ptr(out),
                                          _lib.stream_ptr(codes.device)), "carekv_dequantize_rows")
    return out


def quant_dequant(x: torch.Tensor, bits: int, group: int = 32) -> torch.Tensor:
    """X_hat of the prefill path (layer.py:185-194): quantize, then dequantize
    with the fp16 group scales (not the int8 page scales of the cache)."""
    codes, scale = quantize_rows(x, bits, group)
    return dequantize_rows(codes, scale, group)


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = True,
                      sm_scale: Optional[float] = None, return_lse: bool = False,
                      out: Optional[torch.Tensor] = None):
    """Causal attention over dequantised K/V (layer.py:935-972).

    q: (B, Hq, T, D) or (Hq, T, D) fp16; k, v: (B, Hkv, T, D) or (Hkv, T, D)
    fp16 with Hq a multiple of Hkv (GQA heads are read in place).  Returns
    O like q and, with ``return_lse``, the natural log-sum-exp of each row's
    scaled scores (fp32, (B, Hq, T)): the reference's weights are
    ``exp(q.k * sm_scale - lse)``."""
    squeeze = q.dim() == 3
    if squeeze:
        q, k, v = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)
    q = q.to(torch.float16).contiguous()
    k = k.to(torch.float16).contiguous()
    v = v.to(torch.float16).contiguous()
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    if k.shape != (B, Hkv, T, D) or v.shape != k.shape:
        raise ValueError(f"k/v must be (B, Hkv, T, D) = {(B, Hkv, T, D)}; got {tuple(k.shape)} / {tuple(v.shape)}")
    if out is None:
        out = torch.empty_like(q)
    lse = torch.empty(B, Hq, T, dtype=torch.float32, device=q.device) if return_lse else None
    pp = _lib.PrefillParams(batch=B, n_heads=Hq, n_kv_heads=Hkv, seq_len=T, head_dim=D, causal=int(bool(causal)),
                            sm_scale=float(1.0 / math.sqrt(D)) if sm_scale is None else float(sm_scale))
    lib = _lib.load()
    _lib.check(lib.carekv_prefill_attn(pp, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out),
                                       None if lse is None else _lib.ptr(lse), _lib.stream_ptr(q.device)),
               "carekv_prefill_attn")
    if squeeze:
        out = out[0]
        lse = None if lse is None else lse[0]
    return (out, lse) if return_lse else out


EVAL_KINDS = {"both": 0, "k": 1, "v": 2}


def eval_knobs(read_budget_ratio: float) -> dict:
    """The environment knobs of ``_apply_sparse_prefill_correction_eval``
    (layer.py:375-393), with its defaults and its errors on unknown values."""
    kind = os.environ.get("CAREKV_PREFILL_RESIDUAL_KIND", "both").lower()
    if kind not in EVAL_KINDS:
        raise ValueError(f"Unknown CAREKV_PREFILL_RESIDUAL_KIND={kind}")
    v_score = os.environ.get("CAREKV_V_SCORE", "output_aware").lower()
    if v_score not in {"norm", "output_aware"}:
        raise ValueError(f"Unknown CAREKV_V_SCORE={v_score}")
    return dict(ratio=float(os.environ.get("CAREKV_PREFILL_RESIDUAL_RATIO", str(read_budget_ratio))),
                min_residuals=int(os.environ.get("CAREKV_PREFILL_MIN_RESIDUALS", "1")),
                kind=kind, v_score=v_score, normalize=os.environ.get("CAREKV_SCORE_NORMALIZE", "0") == "1",
                k_corr_scale=float(os.environ.get("CAREKV_K_CORRECTION_SCALE", "0.1")))


def prefill_eval(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_hat: torch.Tensor, v_hat: torch.Tensor,
                 o_base: torch.Tensor, *, ratio: float, min_residuals: int = 1,
                 kind: str = "both", v_score: str = "output_aware", normalize: bool = False,
                 k_corr_scale: float = 0.1, diag_cap: int = 0):
    """``carekv_eval`` prefill correction (layer.py:363-456) of the causal base
    output ``o_base`` (``prefill_attention`` over k_hat / v_hat) from the
    full in-memory residuals k - k_hat, v - v_hat; the base weights are the
    rows' fp32 softmax of q.k_hat / sqrt(D) cast to fp16, recomputed.

    q, o_base: (B, Hq, T, D) or (Hq, T, D) fp16 post-RoPE; k, v, k_hat, v_hat
    (B, Hkv, T, D) or (Hkv, T, D) fp16.
    Returns the corrected output like q and, with ``diag_cap`` > 0, the
    selected token indices of each (head, row), int32 (..., T, diag_cap)
    ascending, -1 padded."""
    squeeze = q.dim() == 3
    if squeeze:
        q, k, v, k_hat, v_hat, o_base = (x.unsqueeze(0) for x in (q, k, v, k_hat, v_hat, o_base))
    q, k, v, k_hat, v_hat, o_base = (x.to(torch.float16).contiguous() for x in (q, k, v, k_hat, v_hat, o_base))
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    for nm, x in (("v", v), ("k_hat", k_hat), ("v_hat", v_hat)):
        if x.shape != k.shape or k.shape != (B, Hkv, T, D):
            raise ValueError(f"{nm} must be (B, Hkv, T, D) = {(B, Hkv, T, D)}; got {tuple(x.shape)}")
    if o_base.shape != q.shape:
        raise ValueError(f"o_base must be {tuple(q.shape)}; got {tuple(o_base.shape)}")
    if kind not in EVAL_KINDS or v_score not in {"norm", "output_aware"}:
        raise ValueError(f"kind {kind!r} / v_score {v_score!r}")
    out = torch.empty_like(q)
    diag = torch.empty(B, Hq, T, diag_cap, dtype=torch.int32, device=q.device) if diag_cap > 0 else None
    pp = _lib.PrefillEvalParams(batch=B, n_heads=Hq, n_kv_heads=Hkv, seq_len=T, head_dim=D, ratio=float(ratio),
                                min_residuals=int(min_residuals), kind=EVAL_KINDS[kind],
                                v_score_norm=int(v_score == "norm"), normalize=int(bool(normalize)),
                                k_corr_scale=float(k_corr_scale), diag_cap=int(diag_cap))
    lib = _lib.load()
    _lib.check(lib.carekv_prefill_eval(pp, *(_lib.ptr(x) for x in (q, k, v, k_hat, v_hat, o_base, out)),
                                       None if diag is None else _lib.ptr(diag), _lib.stream_ptr(q.device)),
               "carekv_prefill_eval")
    if squeeze:
        out = out[0]
        diag = None if diag is None else diag[0]
    return (out, diag) if diag_cap > 0 else out
