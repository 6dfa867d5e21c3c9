"""carekv_decode_attn_static, the decode entry point that allocates nothing
(its workspace is the library's per-GPU static array), called through the C
ABI and held to carekv_decode_attn's output bit for bit (same kernels):
two calls in a row, the second on a smaller input, then a step too large for
the static array, which is refused on the host before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import PAPER_ENV

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _build(care_kv, lens, Hq=8, Hkv=2, D=128, seed=0):
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                              max_pages=max(lens) // 16 + 4, base_bits=3, group_size=32, packed_base=True,
                              scale_quant="int8", store_budget_mode="absolute", store_abs_k=1, store_abs_v=2,
                              read_budget_mode="absolute", read_abs_k=12, read_abs_v=12, route_policy="joint",
                              read_budget_ratio=0.0)
    cache = care_kv.CAREKVCache(cfg, device="cuda", n_seq=len(lens))
    rng = np.random.default_rng(seed)
    for s, T in enumerate(lens):
        K = rng.standard_normal((Hkv, T, D)).astype(np.float16)
        K[:, :, :3] *= np.float16(6.0)
        V = rng.standard_normal((Hkv, T, D)).astype(np.float16)
        cache.write_prefill(0, torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda(), seqs=[s])
    q = torch.from_numpy(rng.standard_normal((len(lens), Hq, D)).astype(np.float16)).cuda()
    return cache, q


def _static_call(care_kv, cache, q, seqs, diag_cap=64):
    """carekv_decode_attn_static through ctypes with caller-built arguments."""
    from care_kv import _lib
    from care_kv.attention import _read_params, default_split_pages
    from care_kv.config import resolve_read_knobs
    lib = _lib.load()
    B, Hq, D = q.shape
    npages = [cache.num_pages(0, 0, s) for s in seqs]
    meta = torch.tensor([seqs, npages], dtype=torch.int32, device="cuda")
    dp = _read_params(cache, 0, resolve_read_knobs(cache.cfg, 0), batch=B, n_heads=Hq, correction=True,
                      split_pages=default_split_pages(max(npages), B * cache.cfg.num_kv_heads),
                      max_pages=max(npages), seq_ptr=meta[0].data_ptr(), np_ptr=meta[1].data_ptr())
    out = torch.empty_like(q)
    diag = torch.empty(B, Hq, diag_cap, dtype=torch.int32, device="cuda")
    rc = lib.carekv_decode_attn_static(ctypes.byref(cache.arena(0)), ctypes.byref(dp), q.data_ptr(), out.data_ptr(),
                                       diag.data_ptr(), diag_cap, _lib.stream_ptr(q.device))
    assert rc == 0, lib.carekv_last_error().decode()
    torch.cuda.synchronize()
    return out, diag


def test_static_decode_matches_workspace_decode(monkeypatch):
    import care_kv
    for k, v in PAPER_ENV.items():
        monkeypatch.setenv(k, v)
    monkeypatch.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    print("no-alloc decode: call 1 (3 sequences, 1500 tokens)", flush=True)
    cache, q = _build(care_kv, [1500, 977, 1200], seed=1)
    ref, rdiag = care_kv.decode_attention(cache, 0, q, diag_cap=64)
    out, diag = _static_call(care_kv, cache, q, [0, 1, 2])
    assert torch.equal(out, ref) and torch.equal(diag, rdiag)
    print("no-alloc decode: call 2 (2 sequences, 300 tokens)", flush=True)
    small, q2 = _build(care_kv, [300, 41], Hq=16, Hkv=4, D=64, seed=2)
    ref2, rdiag2 = care_kv.decode_attention(small, 0, q2, diag_cap=64)
    out2, diag2 = _static_call(care_kv, small, q2, [0, 1])
    assert torch.equal(out2, ref2) and torch.equal(diag2, rdiag2)
    # the Python wrapper's route to the same entry point
    out3 = care_kv.decode_attention(small, 0, q2, no_alloc=True, out=torch.empty_like(q2))
    assert torch.equal(out3, ref2)


def test_static_decode_refuses_steps_beyond_its_array(monkeypatch):
    """A step whose workspace exceeds CAREKV_STATIC_SCRATCH_BYTES fails with
    CAREKV_ESPACE (-3) and a message, on the host, before any launch."""
    import care_kv
    from care_kv import _lib
    from care_kv.attention import _read_params
    from care_kv.config import resolve_read_knobs
    cache, q = _build(care_kv, [64], seed=3)
    lib = _lib.load()
    dp = _read_params(cache, 0, resolve_read_knobs(cache.cfg, 0), batch=200000, n_heads=8, correction=True,
                      split_pages=16, max_pages=cache.cfg.max_pages, seq_ptr=0, np_ptr=0)
    assert lib.carekv_decode_workspace_bytes(ctypes.byref(cache.arena(0)), ctypes.byref(dp)) > _lib.STATIC_SCRATCH_BYTES
    rc = lib.carekv_decode_attn_static(ctypes.byref(cache.arena(0)), ctypes.byref(dp), q.data_ptr(), q.data_ptr(),
                                       None, 0, _lib.stream_ptr(q.device))
    assert rc == -3
    assert b"static scratch" in lib.carekv_last_error()
