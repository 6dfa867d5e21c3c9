"""The reference's quantizer API (quantizer.py:19-383) on the HIP library.

Same names, arguments and results as the reference's functions, for device
tensors: ``quantize`` / ``dequantize`` / ``quantize_and_residual`` (fp16
inputs in fp16 arithmetic, fp32 inputs in fp32 arithmetic, as torch computes
them), ``KQuantizer`` / ``VQuantizer``, the 1-D and 2-D INT2/3/4 bit packers
and ``pack_codes_2d`` / ``unpack_codes_2d``.  The kernels quantize groups of
32 along the last dim with clip_ratio 1.0 (the configuration the cache
uses); other settings raise ``NotImplementedError``.  CPU tensors raise
``CarekvError``: there is no host implementation.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import torch
from torch import Tensor

from . import _lib
from .cache import packed_row_bytes  # noqa: F401  (re-exported, quantizer.py:349-360)
from .prefill import dequantize_rows, quantize_rows


@dataclass
class QuantConfig:
    """quantizer.py:19-24."""
    bits: int = 2
    group_size: int = 64
    symmetric: bool = True
    clip_ratio: float = 1.0


def _check_cfg(cfg: QuantConfig):
    if cfg.group_size != 32 or cfg.clip_ratio != 1.0 or not cfg.symmetric or cfg.bits not in (2, 3, 4):
        raise NotImplementedError(f"the HIP quantizer supports symmetric INT2/3/4 groups of 32 with clip_ratio 1.0 "
                                  f"(got {cfg})")


def quantize(x: Tensor, cfg: QuantConfig) -> Tuple[Tensor, Tensor]:
    """quantizer.py:31-64: (codes int8 like x, scale (..., D / group) in x's
    dtype).  fp16 x runs the fp16 chain (half(max / qmax), half(x / scale),
    round half to even), fp32 x the fp32 chain with the 1e-8 clamp."""
    _check_cfg(cfg)
    _lib.ptr(x)
    D = x.shape[-1]
    if x.dtype == torch.float16:
        return quantize_rows(x, cfg.bits, cfg.group_size)
    if x.dtype != torch.float32:
        raise NotImplementedError(f"quantize of {x.dtype} (fp16 and fp32 are built)")
    x = x.contiguous()
    codes = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scale = torch.empty(*x.shape[:-1], D // 32, dtype=torch.float32, device=x.device)
    lib = _lib.load()
    _lib.check(lib.carekv_quantize_rows_f32(x.data_ptr(), x.numel() // D, D, cfg.bits, 32, codes.data_ptr(),
                                            scale.data_ptr(), _lib.stream_ptr(x.device)), "carekv_quantize_rows_f32")
    return codes, scale


def dequantize(codes: Tensor, scale: Tensor, orig_shape, cfg: QuantConfig) -> Tensor:
    """quantizer.py:67-82: float(code) * float(scale), returned in scale's
    dtype (fp16: half(code * scale))."""
    if cfg.group_size != 32:
        raise NotImplementedError("the HIP dequantizer supports groups of 32")
    _lib.ptr(codes)
    codes = codes.to(torch.int8).reshape(orig_shape)
    if scale.dtype == torch.float16:
        return dequantize_rows(codes, scale.reshape(*orig_shape[:-1], -1), 32)
    if scale.dtype != torch.float32:
        raise NotImplementedError(f"dequantize with {scale.dtype} scales (fp16 and fp32 are built)")
    D = orig_shape[-1]
    codes = codes.contiguous()
    sc = scale.contiguous()
    out = torch.empty(orig_shape, dtype=torch.float32, device=codes.device)
    lib = _lib.load()
    _lib.check(lib.carekv_dequantize_rows_f32(codes.data_ptr(), sc.data_ptr(), codes.numel() // D, D, 32,
                                              out.data_ptr(), _lib.stream_ptr(codes.device)),
               "carekv_dequantize_rows_f32")
    return out


def quantize_and_residual(x: Tensor, cfg: QuantConfig):
    """quantizer.py:85-99: (codes, scale, x - dequantize(codes, scale), x.shape)."""
    codes, scale = quantize(x, cfg)
    x_hat = dequantize(codes, scale, x.shape, cfg)
    return codes, scale, x - x_hat, x.shape


class KQuantizer:
    """quantizer.py:106-120: per-channel-group quantizer for K."""

    def __init__(self, cfg: QuantConfig):
        self.cfg = cfg

    def encode(self, K: Tensor):
        return quantize_and_residual(K, self.cfg)

    def decode(self, codes, scale, shape) -> Tensor:
        return dequantize(codes, scale, shape, self.cfg)


class VQuantizer(KQuantizer):
    """quantizer.py:123-137: per-token quantizer for V (the same group
    quantizer along head_dim)."""


# ------------------------------------------------------------------ bit packing
def _units(bits: int) -> int:
    return 8 if bits == 3 else 8 // bits


def pack_codes_2d(codes: Tensor, bits: int) -> Tensor:
    """quantizer.py:364-372: (T, D) int8 -> (T, packed_row_bytes(D, bits)) int8."""
    if bits not in (2, 3, 4):
        raise ValueError(f"Unsupported base_bits={bits}")
    _lib.ptr(codes)
    codes = codes.to(torch.int8).contiguous()
    T, D = codes.shape
    if D % _units(bits):
        raise AssertionError(f"D={D} must be divisible by {_units(bits)} for INT{bits} packing")
    out = torch.empty(T, D * bits // 8, dtype=torch.int8, device=codes.device)
    lib = _lib.load()
    _lib.check(lib.carekv_pack_codes(codes.data_ptr(), T, D, bits, out.data_ptr(), _lib.stream_ptr(codes.device)),
               "carekv_pack_codes")
    return out


def unpack_codes_2d(packed: Tensor, bits: int, D: int) -> Tensor:
    """quantizer.py:375-383: (T, D*bits/8) int8 -> (T, D) int8, sign-extended."""
    if bits not in (2, 3, 4):
        raise ValueError(f"Unsupported base_bits={bits}")
    _lib.ptr(packed)
    packed = packed.to(torch.int8).contiguous()
    T = packed.shape[0]
    if D % _units(bits) or packed.shape[1] != D * bits // 8:
        raise AssertionError(f"packed rows of {packed.shape[1]} bytes do not hold D={D} INT{bits} codes")
    out = torch.empty(T, D, dtype=torch.int8, device=packed.device)
    lib = _lib.load()
    _lib.check(lib.carekv_unpack_codes(packed.data_ptr(), T, D, bits, out.data_ptr(),
                                       _lib.stream_ptr(packed.device)), "carekv_unpack_codes")
    return out


def _pack_flat(codes: Tensor, bits: int) -> Tensor:
    flat = codes.flatten().to(torch.int8)
    pad = (-flat.numel()) % _units(bits)
    if pad:
        flat = torch.cat([flat, flat.new_zeros(pad)])
    return pack_codes_2d(flat.view(1, -1), bits)[0]


def _unpack_flat(packed: Tensor, numel: int, bits: int) -> Tensor:
    n = packed.numel() * 8 // bits
    return unpack_codes_2d(packed.flatten().view(1, -1), bits, n)[0][:numel]


def pack_int2(codes: Tensor) -> Tensor:
    """quantizer.py:147-160: 1-D codes in [-2, 1], 4 per byte, LSB first."""
    return _pack_flat(codes, 2)


def unpack_int2(packed: Tensor, numel: int) -> Tensor:
    return _unpack_flat(packed, numel, 2)


def pack_int3(codes: Tensor) -> Tensor:
    """quantizer.py:203-226: 1-D codes in [-4, 3], 8 per 24-bit LE word."""
    return _pack_flat(codes, 3)


def unpack_int3(packed: Tensor, numel: int) -> Tensor:
    return _unpack_flat(packed, numel, 3)


def pack_int4(codes: Tensor) -> Tensor:
    """quantizer.py:175-187: 1-D codes in [-8, 7], low nibble = even index."""
    return _pack_flat(codes, 4)


def unpack_int4(packed: Tensor, numel: int) -> Tensor:
    return _unpack_flat(packed, numel, 4)


def pack_int2_2d(codes: Tensor) -> Tensor:
    return pack_codes_2d(codes, 2)


def unpack_int2_2d(packed: Tensor, D: int) -> Tensor:
    return unpack_codes_2d(packed, 2, D)


def pack_int3_2d(codes: Tensor) -> Tensor:
    return pack_codes_2d(codes, 3)


def unpack_int3_2d(packed: Tensor, D: int) -> Tensor:
    return unpack_codes_2d(packed, 3, D)


def pack_int4_2d(codes: Tensor) -> Tensor:
    return pack_codes_2d(codes, 4)


def unpack_int4_2d(packed: Tensor, D: int) -> Tensor:
    return unpack_codes_2d(packed, 4, D)
