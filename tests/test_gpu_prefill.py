"""Prefill-side HIP kernels vs the CPU oracle (needs a GPU).

* ``carekv_quantize_rows`` + ``carekv_dequantize_rows`` reproduce
  ``quantize`` / ``dequantize`` (quantizer.py:31-82) bit for bit.
* ``carekv_prefill_attn`` reproduces ``_causal_attention_pure``
  (layer.py:935-972): every output element within max-abs 2e-3 (or one fp16
  ulp of the reference where that is larger) and the output within
  relative L2 1e-2 of the oracle; for V with per-channel log-normal scales
  (config 4) the absolute bar is 2e-3 times the rms of V; the log-sum-exp
  within 1e-3 absolute.
"""
import math

import numpy as np
import pytest
import torch

from oracle import quant as Q
from oracle.attention import causal_attention_pure

pytestmark = pytest.mark.gpu

F16, F32 = np.float16, np.float32


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _inputs(B, Hq, Hkv, T, D, seed, v_lognormal=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, T, D, generator=g).half()
    k = torch.randn(B, Hkv, T, D, generator=g).half()
    v = torch.randn(B, Hkv, T, D, generator=g)
    if v_lognormal:  # per-channel log-normal scales (sigma 1), as config 4
        v = v * torch.exp(torch.randn(1, Hkv, 1, D, generator=g))
    return q, k, v.half()


def _check(out, ref, v, lognormal=False):
    ulp = np.spacing(np.abs(ref.astype(F16))).astype(F32)
    out = out.astype(F32)
    ref = ref.astype(F32)
    vs = max(1.0, float(np.sqrt(np.mean(v.astype(F32) ** 2)))) if lognormal else 1.0
    err = np.abs(out - ref)
    bound = np.maximum(2e-3 * vs, ulp)
    assert np.isfinite(out).all()
    assert (err <= bound).all(), f"max err {err.max():.3e}, worst ratio {(err / bound).max():.2f}"
    rel = float(np.linalg.norm(out - ref) / max(np.linalg.norm(ref), 1e-30))
    assert rel <= 1e-2, rel


PREFILL_CASES = [
    # B, Hq, Hkv, T, D, causal, lognormal V
    (1, 4, 2, 1, 64, True, False),
    (2, 4, 1, 130, 128, True, False),
    (1, 2, 2, 333, 128, True, False),
    (1, 8, 2, 200, 64, True, False),
    (1, 2, 1, 150, 128, False, False),
    (2, 2, 2, 257, 128, True, True),
]


@pytest.mark.parametrize("case", PREFILL_CASES, ids=[f"B{c[0]}H{c[1]}/{c[2]}T{c[3]}D{c[4]}{'c' if c[5] else 'n'}"
                                                      f"{'L' if c[6] else ''}" for c in PREFILL_CASES])
def test_prefill_attention_vs_oracle(case):
    import care_kv
    B, Hq, Hkv, T, D, causal, logn = case
    print(f"prefill case B={B} Hq={Hq} Hkv={Hkv} T={T} D={D} causal={causal}", flush=True)
    q, k, v = _inputs(B, Hq, Hkv, T, D, 11 + T, logn)
    out, lse = care_kv.prefill_attention(q.cuda(), k.cuda(), v.cuda(), causal=causal, return_lse=True)
    torch.cuda.synchronize()
    out, lse = out.cpu().numpy(), lse.cpu().numpy()
    for b in range(B):
        ref, ref_lse = causal_attention_pure(q[b].numpy(), k[b].numpy(), v[b].numpy(), causal=causal)
        _check(out[b], ref, v[b].numpy(), logn)
        assert np.abs(lse[b] - ref_lse).max() < 1e-3


def test_prefill_attention_long_sequence_rows():
    """T = 4096 (32 query blocks, 128 key tiles): sampled rows at block and
    tile boundaries against the oracle restricted to those rows."""
    import care_kv
    B, Hq, Hkv, T, D = 1, 2, 1, 4096, 128
    print("prefill long rows T=4096", flush=True)
    q, k, v = _inputs(B, Hq, Hkv, T, D, 99)
    out = care_kv.prefill_attention(q.cuda(), k.cuda(), v.cuda()).cpu().numpy()
    rows = [0, 1, 31, 32, 63, 64, 95, 127, 128, 2047, 2048, 4032, 4095]
    ref, _ = causal_attention_pure(q[0].numpy(), k[0].numpy(), v[0].numpy(), rows=rows)
    _check(out[0][:, rows], ref, v[0].numpy())


def test_prefill_attention_is_causal():
    """Changing tokens after t leaves rows <= t bit-identical."""
    import care_kv
    q, k, v = _inputs(1, 2, 2, 300, 128, 7)
    o1 = care_kv.prefill_attention(q.cuda(), k.cuda(), v.cuda())
    k2, v2 = k.clone(), v.clone()
    k2[:, :, 200:] = 3.0
    v2[:, :, 200:] = -5.0
    o2 = care_kv.prefill_attention(q.cuda(), k2.cuda(), v2.cuda())
    assert torch.equal(o1[:, :, :200], o2[:, :, :200])
    assert not torch.equal(o1[:, :, 200:], o2[:, :, 200:])


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_quant_dequant_bit_exact(bits):
    """X_hat of the prefill path: fp16 quantize, then half(code * fp16 scale)."""
    import care_kv
    g = torch.Generator().manual_seed(bits)
    x = (torch.randn(300, 128, generator=g) * torch.exp(torch.randn(1, 128, generator=g))).half()
    codes, scale = care_kv.quantize_rows(x.cuda(), bits)
    xh = care_kv.dequantize_rows(codes, scale).cpu().numpy()
    rc, rs = Q.quantize(x.numpy(), bits, 32)
    assert np.array_equal(codes.cpu().numpy(), rc)
    assert np.array_equal(scale.cpu().numpy().view(np.uint16), rs.astype(F16).view(np.uint16))
    ref = Q.dequantize(rc, rs, 32).astype(F16)
    assert np.array_equal(xh.view(np.uint16), ref.view(np.uint16))
