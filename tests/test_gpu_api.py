"""The reference's package interface on the HIP library (needs a GPU):
``CAREKVCache`` page / slot methods, ``ResidualStoreManager.process_page``,
``ResidualRouter.route``, ``CAREKVAttention``, ``apply_slot_corrections``,
the quantizer and packers of ``__init__.py:15-62`` and the debug read
counters (layer.py:90-126).

Bars: bytes equal to the reference goldens (write_base + process_page
replaying the golden store, write_base + append_to_page replaying the golden
append) and to the oracle (codes, scales, packed bytes, 4-bit slots); route
selections equal the oracle's up to epsilon ties (2e-3 relative, the sketch
proxy); outputs within max-abs 2e-3 of the oracle; read counters equal to
the selections' sizes.
"""
import math

import numpy as np
import pytest
import torch

from helpers import PAPER_ENV, load_golden
from oracle import quant as Q
from oracle.attention import decode_attention as oracle_decode
from oracle.cache import OCache, OCfg
from oracle.check import decode_diag, oracle_candidates, oracle_selection, ties_explain
from oracle.store import write_pages_for_kv_head

pytestmark = pytest.mark.gpu
F16, F32 = np.float16, np.float32


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


@pytest.fixture
def paper_env(monkeypatch):
    for k, v in PAPER_ENV.items():
        monkeypatch.setenv(k, v)
    monkeypatch.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    return monkeypatch


@pytest.mark.parametrize("tag", ["abs", "ratio"])
def test_write_base_and_process_page_replay_store_golden(paper_env, tag):
    """The golden store's page loop (layer.py:254-332) through the reference
    methods: alloc_page, quantize, CAREKVCache.write_base,
    ResidualStoreManager.process_page -- the cache bytes equal store_d128.npz."""
    import care_kv
    from test_gpu_parity import compare_cache_to_golden
    g = load_golden("store_d128.npz")
    kw = dict(num_layers=1, num_heads=2, num_kv_heads=2, head_dim=128, page_size=16, max_pages=8, base_bits=3,
              group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32, packed_base=True,
              scale_quant="int8", compat=True)
    kw.update(dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4) if tag == "abs"
              else dict(store_budget_mode="ratio", store_budget_ratio=0.03))
    cfg = care_kv.CacheConfig(**kw)
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    sm = care_kv.ResidualStoreManager(cfg, 0, "cuda")
    qc = care_kv.QuantConfig(bits=3, group_size=32)
    K, V = torch.from_numpy(g["K"]).cuda(), torch.from_numpy(g["V"]).cuda()
    T, ps = K.shape[1], 16
    n_pages = math.ceil(T / ps)
    for h in range(2):
        for p in range(n_pages):
            t0, t1 = p * ps, min((p + 1) * ps, T)
            nv = t1 - t0
            Kp = torch.nn.functional.pad(K[h, t0:t1], (0, 0, 0, ps - nv))
            Vp = torch.nn.functional.pad(V[h, t0:t1], (0, 0, 0, ps - nv))
            pid = cache.alloc_page(0, h)
            Kc, Ks = care_kv.quantize(Kp, qc)
            Vc, Vs = care_kv.quantize(Vp, qc)
            cache.write_base(0, h, pid, Kc, Ks, Vc, Vs, num_valid=nv)
            meta = sm.process_page(cache, h, pid, Kp, Vp, Kc, Ks, Vc, Vs, token_start=t0, num_valid=nv,
                                   is_recent=p >= n_pages - 4, is_sink=t0 < 4)
            assert meta is not None and meta.num_tokens == nv and meta.token_start == t0
    torch.cuda.synchronize()
    compare_cache_to_golden(cache, g, tag + "_")


def test_write_base_and_append_to_page_replay_append_golden(paper_env):
    """golden_append: write_base of a 10-row page, six append_to_page rows
    into it (fixed master), a fresh page with five appended rows (zero
    master, cfg.compat) -- codes and scales read back equal append_d64.npz."""
    import care_kv
    g = load_golden("append_d64.npz")
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=1, num_kv_heads=1, head_dim=64, page_size=16, max_pages=4,
                              base_bits=3, group_size=32, packed_base=True, scale_quant="int8",
                              store_budget_mode="absolute", compat=True)
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    qc = care_kv.QuantConfig(bits=3, group_size=32)
    X = torch.from_numpy(g["X"]).cuda()
    page = torch.cat([X[:, :10], torch.zeros(2, 6, 64, dtype=X.dtype, device=X.device)], 1)
    Kc, Ks = care_kv.quantize(page[0], qc)
    Vc, Vs = care_kv.quantize(page[1], qc)
    p0 = cache.alloc_page(0, 0)
    cache.write_base(0, 0, p0, Kc, Ks, Vc, Vs, num_valid=10)
    for i in range(10, 16):
        kc, ks = care_kv.quantize(X[0, i:i + 1], qc)
        vc, vs = care_kv.quantize(X[1, i:i + 1], qc)
        assert cache.append_to_page(0, 0, p0, kc[0], ks[0], vc[0], vs[0]) == i
    p1 = cache.alloc_page(0, 0)
    for i in range(16, 21):
        kc, ks = care_kv.quantize(X[0, i:i + 1], qc)
        vc, vs = care_kv.quantize(X[1, i:i + 1], qc)
        cache.append_to_page(0, 0, p1, kc[0], ks[0], vc[0], vs[0])
    kc, ks, vc, vs, lens = cache.read_base_concat(0, 0, [p0, p1])
    assert lens == g["read_lens"].tolist()
    assert np.array_equal(kc.cpu().numpy(), g["read_Kc"]) and np.array_equal(vc.cpu().numpy(), g["read_Vc"])
    assert np.array_equal(ks.cpu().numpy(), g["read_Ks"]) and np.array_equal(vs.cpu().numpy(), g["read_Vs"])
    # a page list out of order reads the pages in list order (cache.py:744-770)
    kc2, ks2, _, _, lens2 = cache.read_base_concat(0, 0, [p1, p0])
    assert lens2 == lens[::-1]
    assert torch.equal(kc2, torch.cat([kc[16:], kc[:16]])) and torch.equal(ks2, torch.cat([ks[16:], ks[:16]]))
    # read_base: every row of the pages, padding included (cache.py:776-798)
    kb, ksb, _, _ = cache.read_base(0, 0, [p0, p1])
    assert kb.shape == (32, 64) and torch.equal(kb[:16], kc[:16]) and torch.equal(kb[16:21], kc[16:21])
    assert torch.equal(ksb[:16], ks[:16])
    # the reference's slot free lists: ascending fresh ids, freed ids last
    assert cache.alloc_k_slot() == 0 and cache.alloc_k_slot() == 1
    cache.free_k_slot(0)
    assert cache.alloc_k_slot() == 2


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_quantizer_and_packers_match_oracle(bits):
    """quantize / dequantize (fp16 and fp32 chains), pack_codes_2d /
    unpack_codes_2d, the 1-D pack_int* of an odd length and pack_4bit /
    unpack_4bit against the oracle, byte for byte."""
    import care_kv
    rng = np.random.default_rng(bits)
    X = (rng.standard_normal((37, 128)) * np.exp(rng.standard_normal((1, 128)))).astype(F16)
    X[3, :32] = 0  # an all-zero group
    qc = care_kv.QuantConfig(bits=bits, group_size=32)
    for dt in (F16, F32):
        x = torch.from_numpy(X.astype(dt)).cuda()
        c, s = care_kv.quantize(x, qc)
        rc, rs = Q.quantize(X.astype(dt), bits, 32)
        assert np.array_equal(c.cpu().numpy(), rc), dt
        assert np.array_equal(s.cpu().numpy().astype(dt).view(np.uint16 if dt == F16 else np.uint32),
                              rs.astype(dt).view(np.uint16 if dt == F16 else np.uint32)), dt
        xh = care_kv.dequantize(c, s, x.shape, qc).cpu().numpy()
        ref = Q.dequantize(rc, rs.astype(dt), 32).astype(dt)
        assert np.array_equal(xh.view(np.uint16 if dt == F16 else np.uint32),
                              ref.view(np.uint16 if dt == F16 else np.uint32)), dt
        codes, scale, resid, shape = care_kv.quantize_and_residual(x, qc)
        assert shape == x.shape and torch.equal(resid, x - care_kv.dequantize(codes, scale, x.shape, qc))
    lo, hi = -(2 ** (bits - 1)), 2 ** (bits - 1) - 1
    codes = rng.integers(lo, hi + 1, size=(21, 128)).astype(np.int8)
    cd = torch.from_numpy(codes).cuda()
    pk = care_kv.pack_codes_2d(cd, bits)
    assert np.array_equal(pk.cpu().numpy(), Q.pack_codes_2d(codes, bits))
    assert torch.equal(care_kv.unpack_codes_2d(pk, bits, 128), cd)
    flat = codes.ravel()[:101]
    p1 = {2: care_kv.pack_int2, 3: care_kv.pack_int3, 4: care_kv.pack_int4}[bits](torch.from_numpy(flat).cuda())
    assert np.array_equal(p1.cpu().numpy(), {2: Q.pack_int2, 3: Q.pack_int3, 4: Q.pack_int4}[bits](flat))
    u1 = {2: care_kv.unpack_int2, 3: care_kv.unpack_int3, 4: care_kv.unpack_int4}[bits](p1, 101)
    assert np.array_equal(u1.cpu().numpy(), flat)
    for dt in (F32, F16):
        r = (rng.standard_normal(512) * 0.3).astype(dt)
        pk4, s4 = care_kv.pack_4bit(torch.from_numpy(r).cuda())
        rp, rsc = Q.pack_4bit(r.astype(F32)) if dt == F32 else (None, None)
        if dt == F32:
            assert np.array_equal(pk4.cpu().numpy(), rp) and s4.cpu().numpy()[0] == rsc
        un = care_kv.unpack_4bit(pk4, s4, 512).cpu().numpy()
        assert np.abs(un - r.astype(F32)).max() <= float(s4.cpu().numpy()[0]) * 0.51 + 1e-6


def test_router_attention_and_read_counters_match_oracle(paper_env):
    """ResidualRouter.route, CAREKVAttention.forward, apply_slot_corrections
    and CAREKVMultiHeadAttention (compat: the router's sketch-proxy score,
    the reference's per-query decode path) against the oracle, and the
    device read counters against the selection sizes."""
    import care_kv
    paper_env.setenv("CAREKV_DEBUG_STATS", "1")
    rng = np.random.default_rng(21)
    D, Hq, Hkv, T = 64, 8, 2, 300
    K = rng.standard_normal((Hkv, T, D)).astype(F16)
    V = rng.standard_normal((Hkv, T, D)).astype(F16)
    K[:, :, rng.permutation(D)[:3]] *= F16(6.0)
    Qh = rng.standard_normal((Hq, D)).astype(F16)
    common = dict(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16, max_pages=T // 16 + 4,
                  base_bits=3, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                  read_budget_mode="absolute", read_abs_k=5, read_abs_v=5, route_policy="joint",
                  store_budget_mode="absolute", store_abs_k=2, store_abs_v=2)
    oc = OCache(OCfg(**common))
    for h in range(Hkv):
        write_pages_for_kv_head(oc, 0, h, K[h], V[h])
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.03, compat=True, **common)
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    cache.write_prefill(0, torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda())
    odiag = {}
    ref = oracle_decode(oc, 0, Qh, k_mode="exact", kind="both", k_corr_scale=1.0, score_normalize=True,
                        kscore_live=False, diag=odiag)
    router = care_kv.ResidualRouter(cfg, 0, "cuda")
    attn = care_kv.CAREKVAttention(cfg, 0, "cuda")
    grp = Hq // Hkv
    care_kv.reset_debug_stats()
    n_k = n_v = 0
    for h in range(Hkv):
        Kc, Vc = oracle_candidates(oc, 0, h, oc.next_page[0][h])
        refs = oracle_selection(odiag[h], Kc, Vc)
        pids = cache.all_page_ids(0, h)
        for j in range(grp):
            q = torch.from_numpy(Qh[h * grp + j]).cuda()
            ks, vs = router.route(cache, h, pids, q, kind="both", score_normalize=True)
            mine = {(0, p, c) for p, c, _ in ks} | {(1, p, b) for p, b, _ in vs}
            assert ties_explain(mine, refs[j], odiag[h], Kc, Vc, j, eps=2e-3), (h, j, sorted(mine ^ refs[j]))
            n_k += len(ks)
            n_v += len(vs)
            for p, c, slot in ks:
                assert slot == int(cache.k_slot[0, h, 0, p, c])
            o = attn.forward(cache, h, q, kind="both", k_corr_scale=1.0, score_normalize=True)
            assert np.abs(o.float().cpu().numpy() - ref[h * grp + j].astype(F32)).max() <= 2e-3
            ob = care_kv.decode_attention(cache, 0, torch.from_numpy(Qh).cuda()[None], correction=False)[0, h * grp + j]
            d = care_kv.apply_slot_corrections(cache, cfg, router, 0, h, pids, q, O_base=ob.float(), kind="both",
                                               k_corr_scale=1.0, score_normalize=True)
            assert torch.equal((ob.float() + d).half(), o.half())
    st = care_kv.get_debug_stats()
    # route and CAREKVAttention each ran the correction once per query; the
    # apply_slot_corrections call once more
    assert st["k_slots_read"] == 3 * n_k and st["v_slots_read"] == 3 * n_v and st["n_queries"] == 3 * Hq
    mha = care_kv.CAREKVMultiHeadAttention(cfg, 0, "cuda")
    out = mha.forward(cache, torch.from_numpy(Qh).cuda(), kind="both", k_corr_scale=1.0, score_normalize=True)
    assert np.abs(out.float().cpu().numpy() - ref.astype(F32)).max() <= 2e-3
    care_kv.reset_debug_stats()
    assert care_kv.get_debug_stats()["k_slots_read"] == 0


def test_page_lists_and_debug_norms(paper_env):
    """CAREKVAttention.forward over page lists other than 0..n-1 (a subset
    in shuffled order, attention.py:979-990) against the oracle's decode over
    the same list, and apply_slot_corrections' debug dict: slot reads, and
    the norms of the linear V term, the linear K term, the applied
    correction and O_base (attention.py:358-372) against an fp64
    recomputation from the oracle cache's rows and slots for the GPU's
    selection."""
    import care_kv
    rng = np.random.default_rng(31)
    D, Hq, Hkv, T = 64, 8, 2, 200
    K = rng.standard_normal((Hkv, T, D)).astype(F16)
    V = rng.standard_normal((Hkv, T, D)).astype(F16)
    K[:, :, rng.permutation(D)[:3]] *= F16(6.0)
    Qh = rng.standard_normal((Hq, D)).astype(F16)
    common = dict(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16, max_pages=T // 16 + 4,
                  base_bits=3, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                  read_budget_mode="absolute", read_abs_k=4, read_abs_v=4, route_policy="joint",
                  store_budget_mode="absolute", store_abs_k=2, store_abs_v=2)
    oc = OCache(OCfg(**common))
    for h in range(Hkv):
        write_pages_for_kv_head(oc, 0, h, K[h], V[h])
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.03, compat=True, **common)
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    cache.write_prefill(0, torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda())
    lists = {0: [7, 2, 11, 0, 5], 1: [12, 3, 4, 9]}  # page 12 is the partial last page
    ref = oracle_decode(oc, 0, Qh, page_ids_by_kvh=lists, k_mode="exact", kind="both", k_corr_scale=1.0,
                        score_normalize=True, kscore_live=False)
    attn = care_kv.CAREKVAttention(cfg, 0, "cuda")
    router = care_kv.ResidualRouter(cfg, 0, "cuda")
    grp = Hq // Hkv
    for h, pids in lists.items():
        for j in range(grp):
            q = torch.from_numpy(Qh[h * grp + j]).cuda()
            o = attn.forward(cache, h, q, page_ids=pids, kind="both", k_corr_scale=1.0, score_normalize=True)
            assert np.abs(o.float().cpu().numpy() - ref[h * grp + j].astype(F32)).max() <= 2e-3, (h, j)
            # the debug norms of one corrected query, recomputed in fp64
            stats = {}
            ob, _ = care_kv.attention.single_query_decode(cache, 0, h, q, page_ids=pids, correction=False)
            d = care_kv.apply_slot_corrections(cache, cfg, router, 0, h, pids, q, O_base=ob.float(), kind="both",
                                               k_corr_scale=0.5, score_normalize=True, debug_stats=stats)
            _, sel = care_kv.attention.single_query_decode(cache, 0, h, q, page_ids=pids, kind="both",
                                                           k_corr_scale=0.5, score_normalize=True, want_diag=True)
            Kc, Ks, Vc, Vs, lens = oc.read_base_concat(0, h, pids)
            Kf = Q.dequantize(Kc, Ks, 32).astype(np.float64)
            Vf = Q.dequantize(Vc, Vs, 32).astype(np.float64)
            qf = Qh[h * grp + j].astype(np.float64)
            s = Kf @ qf / math.sqrt(D)
            a = np.exp(s - s.max())
            a /= a.sum()
            off = np.concatenate([[0], np.cumsum(lens)])
            obf = ob.float().cpu().numpy().astype(np.float64)
            dV, dK = np.zeros(D), np.zeros(D)
            for kind_, p, sub in sel:
                i = pids.index(p)
                p0, n = off[i], lens[i]
                meta = oc.meta_table[0][h][p]
                if kind_ == 1:
                    slot = meta.v_residual_slots[sub]
                    R = Q.unpack_4bit(oc.v_residual_buf[slot], oc.v_residual_scale[slot, 0], 4 * D).reshape(4, D)
                    t0, t1 = 4 * sub, min(4 * sub + 4, n)
                    dV += (a[p0 + t0:p0 + t1, None] * R[:t1 - t0]).sum(0)
                else:
                    slot = meta.k_residual_slots[sub]
                    R = Q.unpack_4bit(oc.k_residual_buf[slot], oc.k_residual_scale[slot, 0], 16 * 32).reshape(16, 32)[:n]
                    qd = R.astype(np.float64) @ qf[32 * sub:32 * sub + 32]
                    dK += ((a[p0:p0 + n] * qd)[:, None] * (Vf[p0:p0 + n] - obf)).sum(0)
            nk = sum(1 for c in sel if c[0] == 0)
            assert stats["k_slots_read"] == nk and stats["v_slots_read"] == len(sel) - nk and stats["n_queries"] == 1
            for key, want in (("delta_v_norm_sum", np.linalg.norm(dV)), ("delta_k_norm_sum", 0.5 * np.linalg.norm(dK)),
                              ("delta_o_norm_sum", float(d.norm())), ("o_base_norm_sum", np.linalg.norm(obf))):
                assert abs(stats[key] - want) <= 1e-3 * max(want, 1e-3), (key, stats[key], want)
