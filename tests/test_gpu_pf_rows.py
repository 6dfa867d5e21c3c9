"""The prefill correction's streaming pass over blocks of prompt rows against
the entry-by-entry pass (needs a GPU).

pf_rows_stream_kernel forms the same page records and stored fp16 weights
as decode_stream_kernel in prefill-rows mode (S in the same MFMA reduction
order, the same record arithmetic), so the selections must be equal; the
base output O and its normaliser L are summed per split of this pass's
own size (32 pages, or CAREKV_PF_SPLIT) instead of per split and wave of
the entry pass, so the corrected outputs may differ in the last fp32
bits, i.e. by at most one fp16 ulp (checked at two).  Cases: head_dim 64
and 128, 1 / 4 / 8 query heads per kv head (16, 4, 2 rows per entry), one
and several stored slots per page, exact and linear K corrections, ragged
calls (rows_per_call not a multiple of the rows per entry), and splits of
8 pages (9 splits, the later ones past the short entries' pages).
CAREKV_PF_ROWS=0 selects the entry-by-entry pass; both are held to the
reference goldens in test_gpu_parity.py.
"""
import numpy as np
import pytest
import torch

from helpers import PAPER_ENV

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


@pytest.fixture
def paper_env(monkeypatch):
    for k, v in PAPER_ENV.items():
        monkeypatch.setenv(k, v)
    return monkeypatch


CASES = [
    # T, Hq, Hkv, D, (store K, store V), k_mode, rows_per_call, pages per split (None: the default)
    (1100, 32, 4, 64, None, "exact", 300, None),
    (777, 16, 4, 128, (2, 4), "exact", 257, None),
    (600, 8, 8, 128, None, "linear", 600, None),
    (530, 16, 2, 64, (1, 2), "exact", 101, None),
    (1100, 32, 4, 64, None, "exact", 1100, 8),
]


@pytest.mark.parametrize("case", CASES, ids=[f"T{c[0]}-g{c[1] // c[2]}-D{c[3]}-{c[5]}-sp{c[7]}" for c in CASES])
def test_pf_rows_pass_matches_entry_pass(paper_env, case):
    import care_kv
    T, Hq, Hkv, D, store, k_mode, rpc, split = case
    print(f"pf rows case T={T} Hq={Hq} Hkv={Hkv} D={D} store={store} {k_mode} split={split}", flush=True)
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", k_mode)
    if split is not None:
        paper_env.setenv("CAREKV_PF_SPLIT", str(split))
    dev = torch.device("cuda", 0)
    sb = dict(store_budget_mode="ratio", store_budget_ratio=0.03) if store is None else \
        dict(store_budget_mode="absolute", store_abs_k=store[0], store_abs_v=store[1])
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                              max_pages=T // 16 + 4, base_bits=3, group_size=32, k_channel_group=32,
                              v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8",
                              read_budget_ratio=0.0, read_budget_mode="absolute", read_abs_k=16, read_abs_v=16,
                              route_policy="joint", **sb)
    cache = care_kv.CAREKVCache(cfg, device=dev)
    g = torch.Generator(device=dev).manual_seed(T + D)
    K = torch.randn(Hkv, T, D, generator=g, device=dev)
    K[:, :, :3] *= 5.0
    K = K.half()
    V = torch.randn(Hkv, T, D, generator=g, device=dev).half()
    cache.write_prefill(0, K, V)
    Kh, Vh = care_kv.quant_dequant(K, 3, 32), care_kv.quant_dequant(V, 3, 32)
    Q = torch.randn(T, Hq, D, generator=g, device=dev).half()
    _, lse = care_kv.prefill_attention(Q.transpose(0, 1), Kh, Vh, return_lse=True)
    res = {}
    for mode in ("1", "0"):
        paper_env.setenv("CAREKV_PF_ROWS", mode)
        out, diag = care_kv.prefill_correction(cache, 0, Q, Kh, Vh, lse, diag_cap=64, rows_per_call=rpc)
        torch.cuda.synchronize()
        res[mode] = (out.cpu().numpy(), diag.cpu().numpy())
    (o1, d1), (o0, d0) = res["1"], res["0"]
    assert np.array_equal(d1, d0)
    assert (d1[:, :, 0] >= 0).mean() > 0.5
    a, b = o1.astype(np.float32), o0.astype(np.float32)
    assert np.isfinite(a).all()
    # O/L summed in another fp32 order: error ~ n*eps32 of sum|p v|/L, which
    # is at most max|V| per row; a near-zero output therefore moves by some
    # fp16 ulps of its own while staying far below one ulp of the row's scale.
    ulp = np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float16)).astype(np.float32)
    vmax = float(Vh.abs().max())
    err = np.abs(a - b)
    print(f"max diff {err.max():.3g}, max diff in ulps {(err / ulp).max():.1f}, "
          f"share differing {(err > 0).mean():.4f}", flush=True)
    assert (err <= 2 * ulp + T * 2.0 ** -24 * vmax).all()
