"""Prefill-side operators: exact quantize / dequantize of rows and the
causal attention over dequantised K/V (``CAREKVLayer._causal_attention_pure``,
layer.py:935-972), all on the HIP library."""
from __future__ import annotations

import math
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
