"""Quantizer, bit packing, int8 scale codes and residual-slot packing.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Arithmetic convention: the reference runs torch ops in the dtype of their
inputs; for float16 tensors torch computes each elementwise op in float32 and
rounds the result to float16.  ``_rt`` reproduces that rounding, so feeding a
float16 array gives the reference's float16 chain and a float32 array gives
its float32 chain (checked bit-for-bit against torch in tests).
"""
from __future__ import annotations

import numpy as np

F16 = np.float16
F32 = np.float32


def _rt(a, dt):
    """Round a float32 result to dtype ``dt`` (RNE), like one torch op."""
    return np.asarray(a, dtype=F32).astype(dt)


def qmax_of(bits: int) -> int:
    return 2 ** (bits - 1) - 1


def _nan_to_zero_int8(q):
    q = np.where(np.isnan(q), F32(0.0), q)
    return q.astype(np.int8)


# ---------------------------------------------------------------- quantize
def quantize(x, bits: int, group_size: int, clip_ratio: float = 1.0):
    """Symmetric per-group quantizer.  Follows ``quantizer.py:31-64``.

    Returns (codes int8 with the shape of x, scale with x's dtype and last
    dim D // group_size)."""
    x = np.asarray(x)
    dt = x.dtype
    D = x.shape[-1]
    g = group_size
    assert D % g == 0, (D, g)
    xg = x.reshape(*x.shape[:-1], D // g, g)
    max_abs = np.abs(xg).max(axis=-1, keepdims=True)                       # exact
    max_abs = _rt(max_abs.astype(F32) * F32(clip_ratio), dt)               # quantizer.py:52
    max_abs = _rt(np.maximum(max_abs.astype(F32), F32(1e-8)), dt)          # .clamp(min=1e-8)
    qm = qmax_of(bits)
    scale = _rt(max_abs.astype(F32) / F32(qm), dt)                         # quantizer.py:55
    with np.errstate(invalid="ignore", divide="ignore"):
        q = _rt(xg.astype(F32) / scale.astype(F32), dt)                    # quantizer.py:58
    q = np.rint(q.astype(F32))
    q = np.clip(q, -qm - 1, qm)
    codes = _nan_to_zero_int8(q).reshape(x.shape)                          # NaN -> 0 (torch)
    return codes, scale[..., 0]


def dequantize(codes, scale, group_size: int):
    """``quantizer.py:67-82``: half-or-float(float(code) * float(scale))."""
    codes = np.asarray(codes)
    scale = np.asarray(scale)
    D = codes.shape[-1]
    g = group_size
    xg = codes.reshape(*codes.shape[:-1], D // g, g).astype(F32)
    s = scale[..., None].astype(F32)
    return (xg * s).reshape(codes.shape).astype(scale.dtype)


def kivi_qdq(x, bits: int, per_channel: bool):
    """``kivi_helpers.py:35-59``: symmetric quant-dequant of a (..., T, D)
    array with one scale per channel over T (``quant_dequant_kivi_k``,
    per_channel) or per token over D (``quant_dequant_kivi_v``), in x's
    dtype.  The 1e-8 floor is 0 in float16, so an all-zero channel (or a
    zero component of a single-row K) gives 0/0 = NaN and stays NaN through
    round and clamp (torch propagates it) -- unlike ``quantize``, whose int8
    cast turns it into 0."""
    x = np.asarray(x)
    dt = x.dtype
    qm = float(qmax_of(bits))
    axis = -2 if per_channel else -1
    m = np.abs(x).max(axis=axis, keepdims=True)                            # exact
    scale = _rt(m.astype(F32) / F32(qm), dt)
    scale = np.maximum(scale, np.asarray(1e-8).astype(dt))                 # .clamp(min=1e-8) in dt
    with np.errstate(invalid="ignore", divide="ignore"):
        q = _rt(x.astype(F32) / scale.astype(F32), dt)
    q = np.rint(q.astype(F32))
    q = np.where(np.isnan(q), q, np.clip(q, -qm - 1, qm))
    return _rt(q * scale.astype(F32), dt)


def kivi_codes(x, bits: int, per_channel: bool):
    """The packed KIVI form of ``kivi_qdq`` (no reference counterpart; the
    reference keeps only the dequantised fp16 side buffer): (codes int8 of
    x's shape, scales of shape (..., 1, D) per channel or (..., T, 1) per
    token) with the quotient, rint and clamp of ``kivi_qdq`` and a NaN
    quotient coded 0; a scale whose max |x| is 0 is NaN, so that
    half(code * scale) reproduces kivi_qdq's NaNs there.  A nonzero max |x|
    whose scale is 0 in fp16 (below 2^-25 qmax) codes its exact zeros as 0
    where kivi_qdq gives NaN: that case is left out of the packed form."""
    x = np.asarray(x)
    dt = x.dtype
    qm = float(qmax_of(bits))
    axis = -2 if per_channel else -1
    m = np.abs(x).max(axis=axis, keepdims=True)
    scale = _rt(m.astype(F32) / F32(qm), dt)
    with np.errstate(invalid="ignore", divide="ignore"):
        q = _rt(x.astype(F32) / scale.astype(F32), dt)
    q = np.rint(q.astype(F32))
    codes = np.where(np.isnan(q), 0, np.clip(q, -qm - 1, qm)).astype(np.int8)
    scale = np.where(m == 0, np.asarray(np.nan, dtype=dt), scale)
    return codes, scale


def quantize_and_residual(x, bits, group_size):
    """``quantizer.py:85-99``."""
    codes, scale = quantize(x, bits, group_size)
    x_hat = dequantize(codes, scale, group_size)
    resid = _rt(np.asarray(x).astype(F32) - x_hat.astype(F32), np.asarray(x).dtype)
    return codes, scale, resid


# ---------------------------------------------------------------- packing
def _u8(a):
    return np.asarray(a).astype(np.int8).view(np.uint8)


def pack_int2_2d(codes):
    """``quantizer.py:257-264``: 4 codes per byte, LSB first."""
    T, D = codes.shape
    assert D % 4 == 0
    u = (_u8(codes) & 0x03).reshape(T, D // 4, 4).astype(np.uint8)
    p = u[..., 0] | (u[..., 1] << 2) | (u[..., 2] << 4) | (u[..., 3] << 6)
    return p.astype(np.uint8).view(np.int8)


def unpack_int2_2d(packed, D):
    """``quantizer.py:267-280``."""
    u = _u8(packed)
    T = u.shape[0]
    out = np.stack([(u >> s) & 0x03 for s in (0, 2, 4, 6)], axis=-1).reshape(T, D)
    out = out.astype(np.int16)
    out[out >= 2] -= 4
    return out.astype(np.int8)


def pack_int4_2d(codes):
    """``quantizer.py:283-290``: low nibble = even index."""
    T, D = codes.shape
    assert D % 2 == 0
    u = _u8(codes) & 0x0F
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8).view(np.int8)


def unpack_int4_2d(packed, D):
    """``quantizer.py:293-301``."""
    u = _u8(packed)
    T = u.shape[0]
    out = np.stack([u & 0x0F, (u >> 4) & 0x0F], axis=-1).reshape(T, D).astype(np.int16)
    out[out >= 8] -= 16
    return out.astype(np.int8)


def pack_int3_2d(codes):
    """``quantizer.py:304-324``: 8 codes -> 24-bit LE word sum c_i<<3i -> 3 bytes."""
    T, D = codes.shape
    assert D % 8 == 0
    u = (_u8(codes) & 0x07).astype(np.int64).reshape(T, D // 8, 8)
    word = np.zeros((T, D // 8), dtype=np.int64)
    for i in range(8):
        word |= u[..., i] << (3 * i)
    b = np.stack([word & 0xFF, (word >> 8) & 0xFF, (word >> 16) & 0xFF], axis=-1)
    return b.reshape(T, D * 3 // 8).astype(np.uint8).view(np.int8)


def unpack_int3_2d(packed, D):
    """``quantizer.py:327-343``."""
    u = _u8(packed).astype(np.int64)
    T = u.shape[0]
    u = u.reshape(T, D // 8, 3)
    word = u[..., 0] | (u[..., 1] << 8) | (u[..., 2] << 16)
    out = np.stack([(word >> (3 * i)) & 0x07 for i in range(8)], axis=-1).reshape(T, D)
    out[out >= 4] -= 8
    return out.astype(np.int8)


def packed_row_bytes(D: int, bits: int) -> int:
    """``quantizer.py:350-361``."""
    if bits == 2:
        assert D % 4 == 0
        return D // 4
    if bits == 3:
        assert D % 8 == 0
        return D * 3 // 8
    if bits == 4:
        assert D % 2 == 0
        return D // 2
    raise ValueError(f"Unsupported base_bits={bits}")


def pack_codes_2d(codes, bits):
    return {2: pack_int2_2d, 3: pack_int3_2d, 4: pack_int4_2d}[bits](np.asarray(codes))


def unpack_codes_2d(packed, bits, D):
    return {2: unpack_int2_2d, 3: unpack_int3_2d, 4: unpack_int4_2d}[bits](np.asarray(packed), D)


# 1-D forms (``quantizer.py:147-246``): pad, then reuse the 2-D bit layout.
def pack_int2(codes):
    f = np.asarray(codes).astype(np.int8).ravel()
    f = np.concatenate([f, np.zeros((-f.size) % 4, np.int8)])
    return pack_int2_2d(f[None, :])[0]


def unpack_int2(packed, numel):
    p = np.asarray(packed).ravel()
    return unpack_int2_2d(p[None, :], p.size * 4)[0][:numel]


def pack_int4(codes):
    f = np.asarray(codes).astype(np.int8).ravel()
    f = np.concatenate([f, np.zeros(f.size % 2, np.int8)])
    return pack_int4_2d(f[None, :])[0]


def unpack_int4(packed, numel):
    p = np.asarray(packed).ravel()
    return unpack_int4_2d(p[None, :], p.size * 2)[0][:numel]


def pack_int3(codes):
    f = np.asarray(codes).astype(np.int8).ravel()
    f = np.concatenate([f, np.zeros((-f.size) % 8, np.int8)])
    return pack_int3_2d(f[None, :])[0]


def unpack_int3(packed, numel):
    p = np.asarray(packed).ravel()
    return unpack_int3_2d(p[None, :], p.size // 3 * 8)[0][:numel]


# ---------------------------------------------------------------- int8 scales
def write_scale_page(scale_in):
    """``cache.py:592-604`` (scale_quant=int8): per-page fp16 master + int8 codes."""
    s = np.asarray(scale_in)
    dt = s.dtype
    max_abs = np.abs(s).max()
    max_abs = _rt(np.maximum(F32(max_abs), F32(1e-8)), dt).astype(F32)
    master = F16(F32(max_abs) / F32(127.0))
    with np.errstate(invalid="ignore", divide="ignore"):
        c = s.astype(F32) / F32(master)
    c = np.clip(np.rint(c), -128, 127)
    return _nan_to_zero_int8(c), master


def append_scale_codes(scale_row, master):
    """``cache.py:689-695``: master held fixed (clamped to 1e-8)."""
    m = np.maximum(F32(master), F32(1e-8))
    c = np.clip(np.rint(np.asarray(scale_row).astype(F32) / m), -128, 127)
    return _nan_to_zero_int8(c)


def read_scale(codes, master, out_dtype=F16):
    """``cache.py:713-718``: (float(code) * float(master)).to(fp16)."""
    return (np.asarray(codes).astype(F32) * F32(master)).astype(out_dtype)


# ---------------------------------------------------------------- residual slots
def pack_4bit(x):
    """``residual_store.py:121-136``: codes use the fp32 scale, stored scale is half(s)."""
    x = np.asarray(x, dtype=F32)
    max_abs = max(F32(np.abs(x).max()), F32(1e-8))
    s = F32(F32(max_abs) / F32(7.0))
    codes = np.clip(np.rint(x / s), -8, 7).astype(np.int8).ravel()
    if codes.size % 2:
        codes = np.concatenate([codes, np.zeros(1, np.int8)])
    u = codes.view(np.uint8)
    packed = ((u[0::2] & 0x0F) | ((u[1::2] << 4) & 0xF0)).astype(np.uint8).view(np.int8)
    return packed, F16(s)


def unpack_4bit(packed, scale, numel):
    """``residual_store.py:139-146``."""
    u = _u8(packed)
    inter = np.stack([u & 0x0F, (u >> 4) & 0x0F], axis=-1).ravel()[:numel].astype(np.int16)
    inter[inter > 7] -= 16
    return inter.astype(F32) * F32(scale)


def pack_8bit(x):
    """``residual_store.py:149-156``."""
    x = np.asarray(x, dtype=F32)
    max_abs = max(F32(np.abs(x).max()), F32(1e-8))
    s = F32(F32(max_abs) / F32(127.0))
    codes = np.clip(np.rint(x / s), -128, 127).astype(np.int8).ravel()
    return codes, F16(s)


def unpack_8bit(packed, scale, numel):
    """``residual_store.py:159-161``."""
    return np.asarray(packed).astype(np.int8).ravel()[:numel].astype(F32) * F32(scale)


def pack_residual(x, bits):
    return pack_8bit(x) if bits == 8 else pack_4bit(x)


def unpack_residual(packed, scale, numel, bits):
    return unpack_8bit(packed, scale, numel) if bits == 8 else unpack_4bit(packed, scale, numel)
