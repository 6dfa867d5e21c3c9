"""HIP kernels vs the reference goldens and the CPU oracle (needs a GPU).

Bars: packed codes, int8 scale codes, masters, valid counts, slot ids and
residual slot bytes bit-exact; fp16 error norms / sketches within one fp16
ulp; selected candidates equal except swaps across an epsilon-tie of the
normalised scores (relative 1e-4 of the selection boundary); decode output
within max-abs 2e-3 (or one fp16 ulp of the reference output, where that is
larger) and relative-L2 1e-2 of the reference fp32 path.
"""
import math

import numpy as np
import pytest
import torch

from helpers import (DECODE_CASES, PAPER_ENV, PREFILL_CASES, build_oracle_case, build_oracle_prefill,
                     case_cfg_kwargs, decode_diag, load_golden, oracle_cache_arrays, oracle_candidates,
                     oracle_selection, prefill_cfg_kwargs, ties_explain)
from oracle import quant as Q
from oracle.attention import decode_attention as oracle_decode
from oracle.attention import prefill_stored
from oracle.cache import OCache, OCfg
from oracle.store import decode_append, write_pages_for_kv_head

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
    return monkeypatch


def _ulp_diff(a, b):
    a = np.ascontiguousarray(a).astype(F16).view(np.int16).astype(np.int32)
    b = np.ascontiguousarray(b).astype(F16).view(np.int16).astype(np.int32)
    return int(np.abs(a - b).max()) if a.size else 0


def compare_cache_to_golden(cache, g, prefix=""):
    """Device cache (layer 0, sequence 0) vs golden reference arrays."""
    valid = cache.valid[0, :, 0].cpu().numpy()
    assert np.array_equal(valid, g[prefix + "valid"]), "valid_tokens"
    H, P = valid.shape
    if prefix + "K_hat" in g:
        # fp16 side buffer: K_hat / V_hat rows bit for bit (NaN patterns included)
        for nm, t in (("K_hat", cache.kcodes), ("V_hat", cache.vcodes)):
            mine = t[0, :, 0].cpu().numpy().view(np.uint16)
            ref = g[prefix + nm].view(np.uint16)
            for h in range(H):
                for p in range(P):
                    n = int(valid[h, p])
                    assert np.array_equal(mine[h, p, :n], ref[h, p, :n]), (nm, h, p)
    else:
        for nm, t in (("K_codes", cache.kcodes), ("V_codes", cache.vcodes), ("K_scale", cache.kscale),
                      ("V_scale", cache.vscale)):
            mine = t[0, :, 0].cpu().numpy()
            ref = g[prefix + nm]
            for h in range(H):
                for p in range(P):
                    n = int(valid[h, p])
                    assert np.array_equal(mine[h, p, :n], ref[h, p, :n]), (nm, h, p)
        for nm, t in (("K_master", cache.kmaster), ("V_master", cache.vmaster)):
            mine = t[0, :, 0].cpu().numpy()
            used = valid > 0
            assert np.array_equal(mine[used], g[prefix + nm][used]), nm
    nk, nv = g[prefix + "k_res"].shape[0], g[prefix + "v_res"].shape[0]
    assert cache.next_slot[0].tolist() == [nk, nv], "slot counters"
    assert np.array_equal(cache.k_res[0, :nk].cpu().numpy(), g[prefix + "k_res"])
    assert np.array_equal(cache.k_res_scale[0, :nk].cpu().numpy(), g[prefix + "k_res_scale"][:, 0])
    assert np.array_equal(cache.v_res[0, :nv].cpu().numpy(), g[prefix + "v_res"])
    assert np.array_equal(cache.v_res_scale[0, :nv].cpu().numpy(), g[prefix + "v_res_scale"][:, 0])
    has_meta = cache.has_meta[0, :, 0].cpu().numpy()
    ks = cache.k_slot[0, :, 0].cpu().numpy()
    vs = cache.v_slot[0, :, 0].cpu().numpy()
    ke = cache.k_err[0, :, 0].cpu().numpy()
    ve = cache.v_err[0, :, 0].cpu().numpy()
    sk = cache.k_sketch[0, :, 0].cpu().numpy()
    for h in range(H):
        for p in range(P):
            if g[prefix + "k_slots"][h, p, 0] == -2:
                assert has_meta[h, p] == 0, ("meta present", h, p)
                continue
            assert has_meta[h, p] == 1, ("meta missing", h, p)
            assert ks[h, p].tolist() == g[prefix + "k_slots"][h, p].tolist(), ("k_slots", h, p)
            assert vs[h, p].tolist() == g[prefix + "v_slots"][h, p].tolist(), ("v_slots", h, p)
            assert _ulp_diff(ke[h, p], g[prefix + "k_err"][h, p]) <= 1, ("k_err", h, p)
            assert _ulp_diff(ve[h, p], g[prefix + "v_err"][h, p]) <= 1, ("v_err", h, p)
            assert _ulp_diff(sk[h, p], g[prefix + "k_sketch"][h, p]) <= 1, ("k_sketch", h, p)


# ------------------------------------------------------------------ store
@pytest.mark.parametrize("tag", ["abs", "ratio"])
def test_store_pages_match_reference(paper_env, tag):
    import care_kv
    g = load_golden("store_d128.npz")
    kw = dict(num_layers=1, num_heads=2, num_kv_heads=2, head_dim=128, page_size=16, max_pages=8, base_bits=3,
              group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32, packed_base=True,
              scale_quant="int8", compat=True)
    kw.update(dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4) if tag == "abs"
              else dict(store_budget_mode="ratio", store_budget_ratio=0.03))
    cache = care_kv.CAREKVCache(care_kv.CacheConfig(**kw), device="cuda")
    cache.write_prefill(0, torch.from_numpy(g["K"]).cuda(), torch.from_numpy(g["V"]).cuda())
    torch.cuda.synchronize()
    compare_cache_to_golden(cache, g, tag + "_")


def test_append_matches_reference(paper_env):
    """int8-scale appends into a partial prefill page and a decode-opened page
    (zero master -> zero scales, the reference's behaviour)."""
    import care_kv
    g = load_golden("append_d64.npz")
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=1, num_kv_heads=1, head_dim=64, page_size=16, max_pages=4,
                              base_bits=3, group_size=32, packed_base=True, scale_quant="int8",
                              store_budget_mode="absolute", compat=True)
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    X = torch.from_numpy(g["X"]).cuda()                  # (2, 21, 64): K rows, V rows
    cache.write_prefill(0, X[0:1, :10], X[1:2, :10])
    for i in range(10, 21):
        cache.append(0, X[0:1, i], X[1:2, i])
    kc, ks, vc, vs, lens = cache.read_base_concat(0, 0)
    assert lens == g["read_lens"].tolist()
    assert np.array_equal(kc.cpu().numpy(), g["read_Kc"])
    assert np.array_equal(vc.cpu().numpy(), g["read_Vc"])
    assert np.array_equal(ks.cpu().numpy(), g["read_Ks"])
    assert np.array_equal(vs.cpu().numpy(), g["read_Vs"])


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_kivi_qdq_matches_oracle(bits):
    """carekv_kivi_qdq vs the oracle's quant_dequant_kivi_k / _v, bit for bit
    (NaN included: an all-zero K channel and a zero component of a one-row K
    divide 0 by a zero scale, as in the reference)."""
    import care_kv
    rng = np.random.default_rng(bits)
    X = (rng.standard_normal((3, 70, 128)) * np.exp(rng.standard_normal((1, 1, 128)))).astype(F16)
    X[1, :, 5] = 0
    X[2, 4, 7] = 0
    xd = torch.from_numpy(X).cuda()

    def same(got, ref):  # bit for bit (signed zeros included); NaN where the reference has NaN
        nan = np.isnan(ref.astype(F32))
        return np.array_equal(np.isnan(got.astype(F32)), nan) and \
            np.array_equal(got.view(np.uint16)[~nan], ref.view(np.uint16)[~nan])
    for per_channel in (True, False):
        got = care_kv.kivi_qdq(xd, bits, per_channel).cpu().numpy()
        ref = Q.kivi_qdq(X, bits, per_channel)
        assert same(got, ref), per_channel
    row = xd[2, 4:5]
    got = care_kv.kivi_qdq(row, bits, True).cpu().numpy()
    ref = Q.kivi_qdq(X[2, 4:5], bits, True)
    assert np.isnan(ref[0, 7]) and same(got, ref)


# ------------------------------------------------------------------ decode
def build_gpu_case(g, name):
    import care_kv
    spec = DECODE_CASES[name]
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0, compat=True,
                              **case_cfg_kwargs(g, spec))
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    T, n_app = int(g["T"]), int(g["n_append"])
    K = torch.from_numpy(g["K"]).cuda()
    V = torch.from_numpy(g["V"]).cuda()
    cache.write_prefill(0, K[:, :T], V[:, :T])
    for t in range(T, T + n_app):
        cache.append(0, K[:, t], V[:, t])
    torch.cuda.synchronize()
    return cache, spec


def check_decode(cache, oc, spec, Qh, ref_out, paper_env, k_mode):
    """GPU decode vs oracle selection (epsilon-tie exempt) and reference output."""
    import care_kv
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", k_mode)
    live = spec.get("live", True)
    paper_env.setenv("CAREKV_KSCORE_LIVE", "1" if live else "0")
    q = torch.from_numpy(Qh).cuda()
    out, diag = care_kv.decode_attention(cache, 0, q.unsqueeze(0), diag_cap=1024)
    torch.cuda.synchronize()
    out = out[0].cpu().numpy().astype(F32)
    diag = diag[0].cpu().numpy()
    odiag = {}
    o_out = oracle_decode(oc, 0, Qh, k_mode=k_mode, kind="both", k_corr_scale=0.1, score_normalize=True,
                          kscore_live=live, diag=odiag)
    Hq, Hkv = spec["Hq"], spec["Hkv"]
    grp = Hq // Hkv
    n_mismatch = 0
    for h in range(Hkv):
        d = odiag[h]
        if d.get("sel_k") is None and d.get("sel_v") is None:
            continue
        Kc, Vc = oracle_candidates(oc, 0, h, oc.next_page[0][h])
        ref_rows = oracle_selection(d, Kc, Vc)
        for j in range(grp):
            mine = set(decode_diag(diag[h * grp + j]))
            if mine != ref_rows[j]:
                n_mismatch += 1
                assert ties_explain(mine, ref_rows[j], d, Kc, Vc, j, eps=spec.get("tie_eps", 1e-4)), \
                    (h, j, sorted(mine ^ ref_rows[j]))
    # max-abs 2e-3, or one fp16 ulp of the reference where that is larger
    # (both sides round an fp32 result to fp16: outputs of magnitude >= 2,
    # as with the INT2 KIVI base's wide per-token V scales, can flip an ulp)
    ref32 = ref_out.astype(F32)
    err = np.abs(out - ref32)
    ulp = np.spacing(np.abs(ref_out).astype(F16)).astype(F32)
    assert np.all(err <= np.maximum(2e-3, ulp)), (err.max(), float(np.abs(ref32).max()))
    rel = np.linalg.norm(out - ref_out.astype(F32)) / max(np.linalg.norm(ref_out.astype(F32)), 1e-30)
    assert rel <= 1e-2, rel
    assert n_mismatch * 16 <= max(Hq, 16), n_mismatch  # at most 1 query row in 16 crosses a tie
    return n_mismatch, o_out


@pytest.mark.parametrize("name", list(DECODE_CASES))
def test_decode_matches_reference(paper_env, name):
    g = load_golden(f"decode_{name}.npz")
    cache, spec = build_gpu_case(g, name)
    compare_cache_to_golden(cache, g)
    oc, _ = build_oracle_case(g, name)
    check_decode(cache, oc, spec, g["Q"], g["O"], paper_env, spec["k_mode"])


def test_decode_base_only_matches_reference_decode_step(paper_env):
    """Compat gate: the reference decode_step applies no correction when
    read_budget_ratio == 0 (attention.py:1025); its output is the base path."""
    import care_kv
    g = load_golden("decode_gqa4_d128.npz")
    cache, spec = build_gpu_case(g, "gqa4_d128")
    mha = care_kv.CAREKVMultiHeadAttention(cache.cfg, 0)
    out = mha.forward(cache, torch.from_numpy(g["Q"]).cuda()).cpu().numpy().astype(F32)
    ref = g["decode_step_out"].astype(F32)
    assert np.abs(out - ref).max() <= 2e-3


def test_read_zero_is_base_bit_exact(paper_env):
    import care_kv
    g = load_golden("decode_gqa4_d128.npz")
    cache, spec = build_gpu_case(g, "gqa4_d128")
    q = torch.from_numpy(g["Q"]).cuda().unsqueeze(0)
    base = care_kv.decode_attention(cache, 0, q, correction=False)
    cache.cfg.read_abs_k = cache.cfg.read_abs_v = 0
    corr0 = care_kv.decode_attention(cache, 0, q, correction=True)
    assert torch.equal(base, corr0)


@pytest.mark.parametrize("Hq,Hkv,D,k_mode", [(16, 4, 128, "exact"), (16, 4, 128, "linear"), (16, 2, 64, "exact")])
def test_zero_residuals_correction_is_base_bit_exact(paper_env, Hq, Hkv, D, k_mode):
    """K and V exactly representable in INT3 (integer codes in [-3, 3], every
    32-dim group reaching |3|, so the group scale and the int8 page scale
    decode to 1 and K_hat = K): every stored residual is 0, so whatever the
    router selects adds exactly nothing (dS = 0, e^0 - 1 = 0, R_V = 0) and
    the corrected step (streaming with records, select, apply, combine) must
    give the base-only step's output bit for bit.  This holds the combine's
    O_base to the select kernel's base path (same sums, same rounding)."""
    import care_kv
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", k_mode)
    print(f"zero residuals Hq={Hq} Hkv={Hkv} D={D} {k_mode}", flush=True)
    dev = torch.device("cuda", 0)
    lens = [700, 333, 1024]
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                              max_pages=max(lens) // 16 + 4, base_bits=3, group_size=32, k_channel_group=32,
                              v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8",
                              store_budget_mode="ratio", store_budget_ratio=0.03, read_budget_ratio=0.0,
                              read_budget_mode="absolute", read_abs_k=16, read_abs_v=16, route_policy="joint")
    cache = care_kv.CAREKVCache(cfg, device=dev, n_seq=len(lens))
    g = torch.Generator(device=dev).manual_seed(D + Hq)

    def exact_int3(n):
        x = torch.randint(-3, 4, (Hkv, n, D), generator=g, device=dev).float()
        x.view(Hkv, n, D // 32, 32)[..., 0] = 3.0  # every group's max |x| is 3: scale 1
        return x.half()

    for b, n in enumerate(lens):
        cache.write_prefill(0, exact_int3(n), exact_int3(n), seqs=[b])
    q = torch.randn(len(lens), Hq, D, generator=g, device=dev).half()
    base = care_kv.decode_attention(cache, 0, q, correction=False)
    corr = care_kv.decode_attention(cache, 0, q, correction=True)
    torch.cuda.synchronize()
    assert torch.isfinite(base.float()).all()
    assert torch.equal(base.view(torch.int16), corr.view(torch.int16))


# ------------------------------------------------------------------ prefill carekv_stored
@pytest.mark.parametrize("name", list(PREFILL_CASES))
def test_prefill_correction_matches_reference(paper_env, name):
    """carekv_prefill_correct vs the reference's CAREKVLayer.prefill in
    carekv_stored mode (vectorized correction): the corrected output within
    the decode bar, and each (row, head)'s selection equal to the oracle's
    over the positive-score candidates up to epsilon ties (1e-3 relative:
    the fp16 attention weights are roundings of softmax values, and a weight
    whose fp32 value straddles a rounding point moves one fp16 ulp)."""
    import care_kv
    g = load_golden(f"prefill_{name}.npz")
    spec = PREFILL_CASES[name]
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", spec["k_mode"])
    print(f"prefill correction case {name}", flush=True)
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0,
                              **prefill_cfg_kwargs(g, spec))
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    T, Hq, Hkv = int(g["T"]), spec["Hq"], spec["Hkv"]
    grp = Hq // Hkv
    K = torch.from_numpy(g["K"]).cuda()
    V = torch.from_numpy(g["V"]).cuda()
    cache.write_prefill(0, K, V)
    torch.cuda.synchronize()
    compare_cache_to_golden(cache, g)
    Kh, Vh = care_kv.quant_dequant(K, 3, 32), care_kv.quant_dequant(V, 3, 32)
    Q = torch.from_numpy(g["Q"]).cuda()  # (T, Hq, D)
    Ob, lse = care_kv.prefill_attention(Q.transpose(0, 1), Kh, Vh, return_lse=True)
    base = Ob.transpose(0, 1).cpu().numpy().astype(F32)
    assert np.abs(base - g["O_base"].astype(F32)).max() <= 2e-3
    out, diag = care_kv.prefill_correction(cache, 0, Q, Kh, Vh, lse, diag_cap=256, rows_per_call=64)
    torch.cuda.synchronize()
    out = out.cpu().numpy().astype(F32)
    ref = g["O"].astype(F32)
    err = np.abs(out - ref)
    ulp = np.spacing(np.abs(g["O"])).astype(F32)
    assert np.all(err <= np.maximum(2e-3, ulp)), (err.max(), np.unravel_index(err.argmax(), err.shape))
    # selections against the oracle (the candidates of later pages score 0
    # and are left out on both sides)
    oc, _, okh, ovh = build_oracle_prefill(g, name)
    odiag = {}
    prefill_stored(oc, 0, g["Q"].transpose(1, 0, 2), okh, ovh, k_mode=spec["k_mode"], kind="both",
                   k_corr_scale=0.1, score_normalize=True, kscore_live=True, diag=odiag)
    diag = diag.cpu().numpy()
    n_tie = 0
    for h in range(Hkv):
        d = odiag[h]
        Kc, Vc = oracle_candidates(oc, 0, h, oc.next_page[0][h])
        ref_rows = oracle_selection(d, Kc, Vc)
        sK, sV = d["score_K_r"], d["score_V_r"]
        for gi in range(grp):
            for t in range(T):
                j = gi * T + t
                vals = {c: float(sK[j, i]) for i, c in enumerate(Kc)}
                vals.update({c: float(sV[j, i]) for i, c in enumerate(Vc)})
                mine = {c for c in decode_diag(diag[t, h * grp + gi]) if vals.get(c, 0.0) > 0}
                refs = {c for c in ref_rows[j] if vals[c] > 0}
                if mine != refs:
                    n_tie += 1
                    if spec["policy"] == "joint":
                        assert ties_explain(mine, refs, d, Kc, Vc, j, eps=1e-3), (h, gi, t, sorted(mine ^ refs))
                    else:
                        for kind in (0, 1):
                            a = {c for c in mine if c[0] == kind}
                            b = {c for c in refs if c[0] == kind}
                            assert ties_explain(a, b, d, Kc, Vc, j, eps=1e-3), (h, gi, t, kind)
    assert n_tie <= max(2, T * Hq // 100), n_tie


PREFILL_RANDOM = [
    # D, Hq, Hkv, T, policy, k_mode, store (abs k, abs v), read (k, v)
    (128, 16, 1, 97, "joint", "exact", (1, 1), (5, 5)),       # GQ 16: one row per entry
    (64, 12, 4, 130, "joint", "exact", (2, 4), (4, 6)),       # GQ 3: five rows per entry, 15 columns
    (128, 4, 4, 75, "separate", "exact", (1, 2), (3, 3)),     # MHA: sixteen rows per entry
    (64, 8, 2, 260, "joint", "linear", (1, 1), (16, 16)),     # budget above the visible candidates
    (64, 8, 2, 5, "joint", "exact", (1, 1), (2, 2)),          # one partial page
    (128, 8, 2, 16, "separate", "exact", (2, 4), (3, 3)),     # exactly one page
    (128, 8, 2, 150, "joint", "exact", (2, 4), (6, 6), "kivi_style"),  # the KIVI-style fp16 side buffer
    # 263 pages: the work-group select form (rows past 256 pages) and the
    # later pages' candidate counts over two 256-page chunks of the suffix scan
    (64, 2, 1, 4200, "joint", "exact", (1, 1), (8, 8)),
]


@pytest.mark.parametrize("live", [True, False], ids=["live", "proxy"])
@pytest.mark.parametrize("case", PREFILL_RANDOM, ids=[f"D{c[0]}g{c[1] // c[2]}T{c[3]}{c[4]}{c[5]}"
                                                      + (c[8] if len(c) > 8 else "") for c in PREFILL_RANDOM])
def test_prefill_correction_random_vs_oracle(paper_env, case, live):
    """carekv_prefill_correct vs the oracle's prefill_stored on random
    prompts: GQA widths that pack 1, 5 and 16 rows per entry, a partial last
    page, separate / linear variants and read budgets above the candidates
    a row can see; live: the query-aware K score of correction_impl =
    vectorized, proxy: the router's sketch proxy of correction_impl = cached.
    Selections (positive-score candidates) equal the oracle's up to epsilon
    ties (1e-4 relative for the query-aware score, 2e-3 for the proxy, whose
    1 / margin term amplifies logit rounding), at most 1 row in 16 crossing
    a tie; every output element within max-abs 2e-3 (or one fp16 ulp) of the
    oracle recomputed under the GPU's selection."""
    import care_kv
    from oracle.check import forced_selection
    D, Hq, Hkv, T, pol, kmode, (sk, sv), (rk, rv) = case[:8]
    base = dict(base_bits=2, base_quantizer=case[8]) if len(case) > 8 else dict(base_bits=3)
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", kmode)
    print(f"prefill random case {case} live={live}", flush=True)
    eps = 1e-4 if live else 2e-3
    rng = np.random.default_rng(D + Hq * 7 + T)
    K = rng.standard_normal((Hkv, T, D)).astype(F16)
    V = rng.standard_normal((Hkv, T, D)).astype(F16)
    K[:, :, rng.permutation(D)[:3]] *= F16(6.0)
    Qt = rng.standard_normal((T, Hq, D)).astype(F16)
    common = dict(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16, max_pages=T // 16 + 4,
                  group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                  read_budget_mode="absolute", read_abs_k=rk, read_abs_v=rv, route_policy=pol,
                  store_budget_mode="absolute", store_abs_k=sk, store_abs_v=sv, **base)
    oc = OCache(OCfg(**common))
    hats = [write_pages_for_kv_head(oc, 0, h, K[h], V[h]) for h in range(Hkv)]
    okh, ovh = np.stack([a for a, _ in hats]), np.stack([b for _, b in hats])
    kw = dict(k_mode=kmode, kind="both", k_corr_scale=0.1, score_normalize=True, kscore_live=live)
    odiag = {}
    prefill_stored(oc, 0, Qt.transpose(1, 0, 2), okh, ovh, diag=odiag, **kw)
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0, **common)
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    Kd, Vd = torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda()
    hats = cache.write_prefill(0, Kd, Vd)
    if hats is not None:  # side-buffer base: the K_hat / V_hat the pages hold
        Kh, Vh = hats
    else:
        Kh, Vh = care_kv.quant_dequant(Kd, 3, 32), care_kv.quant_dequant(Vd, 3, 32)
    assert np.array_equal(Kh.cpu().numpy().view(np.uint16), okh.view(np.uint16))
    Q = torch.from_numpy(Qt).cuda()
    _, lse = care_kv.prefill_attention(Q.transpose(0, 1), Kh, Vh, return_lse=True)
    knobs = care_kv.resolve_read_knobs(cfg, 0)
    knobs.kscore_live = live
    out, diag = care_kv.prefill_correction(cache, 0, Q, Kh, Vh, lse, rows_per_call=50, knobs=knobs, diag_cap=64)
    out, diag = out.cpu().numpy().astype(F32), diag.cpu().numpy()
    grp = Hq // Hkv
    n_tie = n_rows = 0
    forced = {}
    for h in range(Hkv):
        d = odiag[h]
        Kc, Vc = oracle_candidates(oc, 0, h, oc.next_page[0][h])
        ref_rows = oracle_selection(d, Kc, Vc)
        sK, sV = d["score_K_r"], d["score_V_r"]
        rows = []
        for gi in range(grp):
            for t in range(T):
                j = gi * T + t
                row = diag[t, h * grp + gi]
                rows.append(row)
                vals = {c: float(sK[j, i]) for i, c in enumerate(Kc)} if sK is not None else {}
                if sV is not None:
                    vals.update({c: float(sV[j, i]) for i, c in enumerate(Vc)})
                mine = {c for c in decode_diag(row) if vals.get(c, 0.0) > 0}
                refs = {c for c in ref_rows[j] if vals.get(c, 0.0) > 0}
                n_rows += 1
                if mine == refs:
                    continue
                n_tie += 1
                kinds = (None,) if pol == "joint" else (0, 1)
                for kind in kinds:
                    a_ = mine if kind is None else {c for c in mine if c[0] == kind}
                    b_ = refs if kind is None else {c for c in refs if c[0] == kind}
                    assert ties_explain(a_, b_, d, Kc, Vc, j, eps=eps), (h, gi, t, kind, sorted(a_ ^ b_))
        forced[h] = forced_selection(rows, Kc, Vc)
    assert n_tie * 16 <= n_rows, (n_tie, n_rows)
    ref = prefill_stored(oc, 0, Qt.transpose(1, 0, 2), okh, ovh, force_sel=forced, **kw).astype(F32)
    err = np.abs(out - ref)
    ulp = np.spacing(np.abs(ref).astype(F16)).astype(F32)
    assert np.all(err <= np.maximum(2e-3, ulp)), (err.max(), np.unravel_index(err.argmax(), err.shape))


# ------------------------------------------------------------------ random shapes vs oracle
RANDOM_CASES = [
    # D, bits, Hq, Hkv, T, n_append, policy, k_mode, store (abs k, abs v) or ratio, read (k, v)
    (128, 3, 8, 2, 700, 5, "joint", "exact", (1, 1), (6, 6)),
    (128, 2, 4, 4, 333, 0, "separate", "exact", (2, 4), (2, 3)),
    (128, 4, 16, 1, 512, 17, "joint", "linear", (2, 2), (8, 4)),
    (64, 3, 32, 4, 256, 3, "joint", "exact", (1, 1), (5, 7)),
    (64, 2, 8, 8, 150, 20, "separate", "linear", (1, 2), (3, 3)),
    (64, 4, 4, 1, 1024, 0, "joint", "exact", (2, 4), (16, 16)),
]


@pytest.mark.parametrize("live", [True, False], ids=["live", "proxy"])
@pytest.mark.parametrize("case", RANDOM_CASES, ids=[f"D{c[0]}b{c[1]}g{c[2]//c[3]}{c[6]}{c[7]}" for c in RANDOM_CASES])
def test_decode_random_vs_oracle(paper_env, case, live):
    """live: the query-aware K score; proxy: the sketch proxy (KSCORE_LIVE=0),
    whose boundary term 1/(s_top - s_t) amplifies logit rounding, so its tie
    band is wider."""
    import care_kv
    D, bits, Hq, Hkv, T, n_app, pol, kmode, (sk, sv), (rk, rv) = case
    eps = 1e-4 if live else 2e-3
    paper_env.setenv("CAREKV_KSCORE_LIVE", "1" if live else "0")
    print(f"random decode case {case} live={live}", flush=True)
    rng = np.random.default_rng(D * 7 + bits * 3 + Hq + T)
    K = (rng.standard_normal((Hkv, T + n_app, D)) * 1.0).astype(F16)
    V = rng.standard_normal((Hkv, T + n_app, D)).astype(F16)
    K[:, :, rng.permutation(D)[:3]] *= F16(6.0)
    Qh = rng.standard_normal((Hq, D)).astype(F16)
    common = dict(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                  max_pages=(T + n_app) // 16 + 4, base_bits=bits, group_size=32, k_channel_group=32,
                  v_token_block=4, sketch_dim=32, read_budget_mode="absolute", read_abs_k=rk, read_abs_v=rv,
                  route_policy=pol, store_budget_mode="absolute", store_abs_k=sk, store_abs_v=sv)
    oc = OCache(OCfg(**common))
    for h in range(Hkv):
        write_pages_for_kv_head(oc, 0, h, K[h, :T], V[h, :T])
    for t in range(T, T + n_app):
        decode_append(oc, 0, K[:, t], V[:, t])
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0, compat=True, **common)
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    Kd, Vd = torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda()
    cache.write_prefill(0, Kd[:, :T], Vd[:, :T])
    for t in range(T, T + n_app):
        cache.append(0, Kd[:, t], Vd[:, t])
    torch.cuda.synchronize()
    # cache bytes equal the oracle's
    assert np.array_equal(cache.valid[0, :, 0].cpu().numpy(), oc.valid_tokens[0])
    assert np.array_equal(cache.k_slot[0, :, 0].cpu().numpy()[cache.has_meta[0, :, 0].cpu().numpy() == 1],
                          np.array([m.k_residual_slots for row in oc.meta_table[0] for m in row if m is not None]))
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", kmode)
    odiag = {}
    o_out = oracle_decode(oc, 0, Qh, k_mode=kmode, kind="both", k_corr_scale=0.1, score_normalize=True,
                          kscore_live=live, diag=odiag)
    out, diag = care_kv.decode_attention(cache, 0, torch.from_numpy(Qh).cuda().unsqueeze(0), diag_cap=1024)
    out = out[0].cpu().numpy().astype(F32)
    err = np.abs(out - o_out.astype(F32))
    assert err.max() <= 2e-3, err.max()
    grp = Hq // Hkv
    diag = diag[0].cpu().numpy()
    n_tie = 0
    for h in range(Hkv):
        d = odiag[h]
        Kc, Vc = oracle_candidates(oc, 0, h, oc.next_page[0][h])
        ref_rows = oracle_selection(d, Kc, Vc)
        for j in range(grp):
            mine = set(decode_diag(diag[h * grp + j]))
            n_tie += mine != ref_rows[j]
            if pol == "joint":
                assert ties_explain(mine, ref_rows[j], d, Kc, Vc, j, eps=eps), (h, j)
            else:
                for kind in (0, 1):
                    a = {c for c in mine if c[0] == kind}
                    b = {c for c in ref_rows[j] if c[0] == kind}
                    assert ties_explain(a, b, d, Kc, Vc, j, eps=eps), (h, j, kind)
    assert n_tie * 16 <= max(Hq, 16), n_tie  # at most 1 query row in 16 crosses a tie


# ------------------------------------------------------------------ INT4 base (config 4's quantizer)
INT4_STORES = {"ratio3": dict(store_budget_mode="ratio", store_budget_ratio=0.03),
               "abs2k4v": dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4)}


def _rounding_allowance(Kh, Vh, Qh, grp):
    """Per (query head, dim): 2^-10 * sum_t a_t |V_hat_t| over the fp32
    softmax weights a of the base attention.  Both the reference and the
    kernel round each weight to fp16 at different points (the reference a,
    the kernel a and then a times the V scale), so an output may differ from
    the reference's by about that much, which matters only where |V| is
    large (per-channel log-normal scales)."""
    out = []
    for h in range(Qh.shape[0]):
        k, v = Kh[h // grp].astype(np.float64), Vh[h // grp].astype(np.float64)
        s = (Qh[h].astype(np.float64) @ k.T) / math.sqrt(k.shape[1])
        a = np.exp(s - s.max())
        out.append(2.0 ** -10 * (a / a.sum()) @ np.abs(v))
    return np.stack(out)


@pytest.mark.parametrize("Hq,Hkv", [(16, 4), (4, 4), (16, 2)], ids=["gq4", "gq1", "gq8"])
@pytest.mark.parametrize("store", sorted(INT4_STORES))
def test_int4_store_and_decode_vs_oracle(paper_env, store, Hq, Hkv):
    """Config 4 names INT4 next to INT3: write_prefill at base_bits 4 and
    D = 128 gives the oracle's page bytes (codes, int8 scale codes,
    masters), metadata, slot ids and 4-bit slot payloads (write_pages_for_kv_head
    on the same rows, pinned by the store goldens at INT3), before and after
    decode appends, for two inputs:
      * decode data (K and V ~N(0, 1), 4 K channels x10, as config 3): the
        corrected decode (exact renormalisation; the 4-query-head streaming
        and apply kernels at GQ 4 and 1, the generic ones at GQ 8) meets the
        decode bar against oracle.decode_attention, selections equal up to
        epsilon ties;
      * config 4's data (per-channel log-normal K and V scales): the base
        decode meets max(2e-3, 1 ulp) plus the weight-rounding allowance.
    """
    import care_kv
    D, bits, T, n_app = 128, 4, 600, 9
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    for data in ("decode", "lognormal"):
        print(f"int4 store+decode store={store} Hq={Hq} Hkv={Hkv} data={data}", flush=True)
        rng = np.random.default_rng(400 + Hq + Hkv + len(store))
        if data == "decode":
            K = rng.standard_normal((Hkv, T + n_app, D))
            K[:, :, rng.permutation(D)[:4]] *= 10.0
            V = rng.standard_normal((Hkv, T + n_app, D))
        else:
            K = rng.standard_normal((Hkv, T + n_app, D)) * np.exp(rng.standard_normal((Hkv, 1, D)))
            V = rng.standard_normal((Hkv, T + n_app, D)) * np.exp(rng.standard_normal((Hkv, 1, D)))
        K, V = K.astype(F16), V.astype(F16)
        Qh = rng.standard_normal((Hq, D)).astype(F16)
        common = dict(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                      max_pages=(T + n_app) // 16 + 4, base_bits=bits, group_size=32, k_channel_group=32,
                      v_token_block=4, sketch_dim=32, read_budget_mode="absolute", read_abs_k=8, read_abs_v=8,
                      route_policy="joint", **INT4_STORES[store])
        oc = OCache(OCfg(**common), max_slots=common["max_pages"] * Hkv * 4)
        for h in range(Hkv):
            write_pages_for_kv_head(oc, 0, h, K[h, :T], V[h, :T])
        cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0, compat=True,
                                  **common)
        cache = care_kv.CAREKVCache(cfg, device="cuda")
        Kd, Vd = torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda()
        cache.write_prefill(0, Kd[:, :T], Vd[:, :T])
        torch.cuda.synchronize()
        compare_cache_to_golden(cache, oracle_cache_arrays(oc))
        for t in range(T, T + n_app):
            decode_append(oc, 0, K[:, t], V[:, t])
            cache.append(0, Kd[:, t], Vd[:, t])
        torch.cuda.synchronize()
        compare_cache_to_golden(cache, oracle_cache_arrays(oc))
        q = torch.from_numpy(Qh).cuda().unsqueeze(0)
        if data == "lognormal":
            out = care_kv.decode_attention(cache, 0, q, correction=False)[0].cpu().numpy().astype(F32)
            ref = oracle_decode(oc, 0, Qh, correction=False).astype(F32)
            kh, vh = [], []
            for h in range(Hkv):
                kc, ks, vc, vs, _ = oc.read_base_concat(0, h, oc.all_page_ids(0, h))
                kh.append(Q.dequantize(kc, ks, 32))
                vh.append(Q.dequantize(vc, vs, 32))
            allow = _rounding_allowance(kh, vh, Qh, Hq // Hkv)
            ulp = np.spacing(np.abs(ref).astype(F16)).astype(F32)
            err = np.abs(out - ref)
            assert np.all(err <= np.maximum(2e-3, ulp + allow)), float((err / np.maximum(2e-3, ulp + allow)).max())
            assert np.linalg.norm(out - ref) <= 1e-2 * np.linalg.norm(ref)
            continue
        odiag = {}
        o_out = oracle_decode(oc, 0, Qh, k_mode="exact", kind="both", k_corr_scale=0.1, score_normalize=True,
                              kscore_live=True, diag=odiag)
        out, diag = care_kv.decode_attention(cache, 0, q, diag_cap=64)
        out = out[0].cpu().numpy().astype(F32)
        ref = o_out.astype(F32)
        grp, diag, n_tie = Hq // Hkv, diag[0].cpu().numpy(), 0
        for h in range(Hkv):
            Kc, Vc = oracle_candidates(oc, 0, h, oc.next_page[0][h])
            ref_rows = oracle_selection(odiag[h], Kc, Vc)
            for j in range(grp):
                mine = set(decode_diag(diag[h * grp + j]))
                n_tie += mine != ref_rows[j]
                assert ties_explain(mine, ref_rows[j], odiag[h], Kc, Vc, j, eps=1e-4), (h, j)
        assert n_tie * 16 <= max(Hq, 16), n_tie
        err = np.abs(out - ref)
        ulp = np.spacing(np.abs(ref).astype(F16)).astype(F32)
        assert np.all(err <= np.maximum(2e-3, ulp)), err.max()
        assert np.linalg.norm(out - ref) <= 1e-2 * np.linalg.norm(ref)


@pytest.mark.parametrize("bits", [4, 3])
def test_config4_store_full_shape(bits):
    """Config 4's store at its full shape (4 sequences, 40 kv heads, 8192
    tokens, D = 128, K and V with per-channel log-normal scales, store ratio
    3%), one batched write_prefill: sampled (sequence, kv head) slices hold
    the oracle's page bytes, metadata and slot payloads (the oracle writes
    each slice alone, so its slot ids are compared relative to the slice's
    first id), and the slot counters equal 4 * 40 * 512 pages' worth."""
    import care_kv
    B, H, T, D = 4, 40, 8192, 128
    print(f"config 4 store bits={bits}", flush=True)
    g = torch.Generator().manual_seed(4)
    K = torch.randn(B, H, T, D, generator=g) * torch.exp(torch.randn(1, H, 1, D, generator=g))
    V = torch.randn(B, H, T, D, generator=g) * torch.exp(torch.randn(1, H, 1, D, generator=g))
    K, V = K.half(), V.half()
    common = dict(num_layers=1, num_heads=H, num_kv_heads=H, head_dim=D, page_size=16, max_pages=T // 16,
                  base_bits=bits, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                  store_budget_mode="ratio", store_budget_ratio=0.03)
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0, compat=True, **common)
    cache = care_kv.CAREKVCache(cfg, device="cuda", n_seq=B)
    cache.write_prefill(0, K.cuda(), V.cuda(), seqs=list(range(B)))
    torch.cuda.synchronize()
    P = T // 16
    assert cache.next_slot.tolist() == [[H * P, H * P]] * B  # one K and one V slot a page (max(1, int(n * 0.03)))
    for s, h in ((0, 0), (3, H - 1), (2, 17)):
        oc = OCache(OCfg(**{**common, "num_heads": 1, "num_kv_heads": 1}), max_slots=P)
        write_pages_for_kv_head(oc, 0, 0, K[s, h].numpy(), V[s, h].numpy())
        ref = oracle_cache_arrays(oc)
        valid = cache.valid[0, h, s].cpu().numpy()
        assert np.array_equal(valid, ref["valid"][0])
        for nm, t in (("K_codes", cache.kcodes), ("V_codes", cache.vcodes), ("K_scale", cache.kscale),
                      ("V_scale", cache.vscale), ("K_master", cache.kmaster), ("V_master", cache.vmaster)):
            assert np.array_equal(t[0, h, s].cpu().numpy(), ref[nm][0]), (nm, s, h)
        ks, vs = cache.k_slot[0, h, s].cpu().numpy(), cache.v_slot[0, h, s].cpu().numpy()
        k0, v0 = int(ks[ks >= 0].min()), int(vs[vs >= 0].min())
        assert (k0, v0) == (h * P, h * P), (s, h, k0, v0)  # kv-head-major slot order within the sequence
        assert np.array_equal(np.where(ks >= 0, ks - k0, -1), ref["k_slots"][0]), (s, h)
        assert np.array_equal(np.where(vs >= 0, vs - v0, -1), ref["v_slots"][0]), (s, h)
        assert np.array_equal(cache.k_res[s, k0:k0 + P].cpu().numpy(), ref["k_res"])
        assert np.array_equal(cache.v_res[s, v0:v0 + P].cpu().numpy(), ref["v_res"])
        assert np.array_equal(cache.k_res_scale[s, k0:k0 + P].cpu().numpy(), ref["k_res_scale"][:, 0])
        assert np.array_equal(cache.v_res_scale[s, v0:v0 + P].cpu().numpy(), ref["v_res_scale"][:, 0])
        for nm, t in (("k_err", cache.k_err), ("v_err", cache.v_err), ("k_sketch", cache.k_sketch)):
            assert _ulp_diff(t[0, h, s].cpu().numpy(), ref[nm][0]) <= 1, (nm, s, h)


def test_batched_sequences_match_single(paper_env):
    """B sequences in one launch == each sequence decoded alone."""
    import care_kv
    rng = np.random.default_rng(11)
    D, Hq, Hkv = 128, 8, 2
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16, max_pages=40,
                              base_bits=3, group_size=32, packed_base=True, scale_quant="int8",
                              store_budget_mode="absolute", store_abs_k=1, store_abs_v=1,
                              read_budget_mode="absolute", read_abs_k=8, read_abs_v=8, route_policy="joint",
                              read_budget_ratio=0.0)
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    lens = [300, 517, 64, 1, 0]  # ragged, a one-token sequence and an empty one
    B = len(lens)
    cache = care_kv.CAREKVCache(cfg, device="cuda", n_seq=B)
    for s, T in enumerate(lens):
        if T == 0:
            continue
        K = torch.from_numpy(rng.standard_normal((Hkv, T, D)).astype(F16)).cuda()
        V = torch.from_numpy(rng.standard_normal((Hkv, T, D)).astype(F16)).cuda()
        cache.write_prefill(0, K, V, seqs=[s])
    q = torch.from_numpy(rng.standard_normal((B, Hq, D)).astype(F16)).cuda()
    both = care_kv.decode_attention(cache, 0, q)
    for s in range(B):
        one = care_kv.decode_attention(cache, 0, q[s:s + 1], seqs=[s])
        assert torch.equal(both[s], one[0])
    assert torch.isfinite(both[3]).all()
    assert torch.count_nonzero(both[4]) == 0  # nothing to attend to: zeros, as an empty softmax sum gives


@pytest.mark.parametrize("D,bits,base,jump", [(64, 3, "uniform", 1.0), (128, 2, "uniform", 1.0),
                                              (64, 2, "kivi_style", 1.0), (64, 3, "uniform", 2.0)])
def test_streaming_store_matches_oracle(paper_env, D, bits, base, jump):
    """The default decode appends (compat=False, no reference counterpart):
    they fill the prompt's partial page and three decode-opened pages, each
    open page without stored slots re-encoded as write_base encodes its rows
    and each fill stored from the true rows against the page's own base,
    reusing the slot ids the page held -- page bytes, slot ids, residual
    bytes and scales equal the oracle's (process_page on the same inputs),
    and the decode over the cache matches the oracle's.  jump: the appended
    rows are that much larger than the prompt's; the prompt's partial page,
    which holds slots, keeps its prefill encoding (master and scale codes)
    until it fills."""
    import care_kv
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    Hq, Hkv, T, n_app = 8, 2, 100, 60
    print(f"streaming store D={D} bits={bits} base={base} jump={jump}", flush=True)
    rng = np.random.default_rng(D + bits)
    K = rng.standard_normal((Hkv, T + n_app, D)).astype(F16)
    V = rng.standard_normal((Hkv, T + n_app, D)).astype(F16)
    K[:, :, rng.permutation(D)[:3]] *= F16(6.0)
    K[:, T:] *= F16(jump)
    V[:, T:] *= F16(jump)
    Qh = rng.standard_normal((Hq, D)).astype(F16)
    common = dict(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                  max_pages=(T + n_app) // 16 + 4, base_bits=bits, group_size=32, k_channel_group=32,
                  v_token_block=4, sketch_dim=32, read_budget_mode="absolute", read_abs_k=6, read_abs_v=6,
                  route_policy="joint", store_budget_mode="absolute", store_abs_k=2, store_abs_v=4,
                  base_quantizer=base)
    oc = OCache(OCfg(**common))
    for h in range(Hkv):
        write_pages_for_kv_head(oc, 0, h, K[h, :T], V[h, :T])
    for t in range(T, T + n_app):
        decode_append(oc, 0, K[:, t], V[:, t], streaming=True, rescale=True)
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0, **common)
    cache = care_kv.CAREKVCache(cfg, device="cuda")  # the default (compat=False): streaming store, re-encoding
    Kd, Vd = torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda()
    cache.write_prefill(0, Kd[:, :T], Vd[:, :T])
    pre_k = cache.k_slot[0, :, 0, T // 16].clone()  # the prompt's partial page
    pre_v = cache.v_slot[0, :, 0, T // 16].clone()
    pre_km = cache.kmaster[0, :, 0, T // 16].clone()
    pre_ks = cache.kscale[0, :, 0, T // 16, :T % 16].clone()
    for t in range(T, T + n_app):
        cache.append(0, Kd[:, t], Vd[:, t])
        if t == T + 2 and jump > 1:  # the prompt page still holds its slots and its prefill encoding
            assert torch.equal(cache.k_slot[0, :, 0, T // 16], pre_k)
            assert torch.equal(cache.kmaster[0, :, 0, T // 16], pre_km)
            assert torch.equal(cache.kscale[0, :, 0, T // 16, :T % 16], pre_ks)
    torch.cuda.synchronize()
    for h in range(Hkv):  # its refill reuses the slot ids it held
        for pre, now in ((pre_k[h], cache.k_slot[0, h, 0, T // 16]), (pre_v[h], cache.v_slot[0, h, 0, T // 16])):
            old_ids = sorted(x for x in pre.tolist() if x >= 0)
            new_ids = sorted(x for x in now.tolist() if x >= 0)
            assert set(old_ids) <= set(new_ids) or set(new_ids) <= set(old_ids), (h, old_ids, new_ids)
    nk, nv = oc.next_k_slot, oc.next_v_slot
    valid = cache.valid[0, :, 0].cpu().numpy()
    assert np.array_equal(valid, oc.valid_tokens[0])
    if base == "uniform":  # the re-encoded pages, byte for byte
        for nm, t, ref in (("K_scale", cache.kscale, oc.base_K_scale), ("V_scale", cache.vscale, oc.base_V_scale),
                           ("K_codes", cache.kcodes, oc.base_K_codes), ("V_codes", cache.vcodes, oc.base_V_codes)):
            mine = t[0, :, 0].cpu().numpy()
            for h in range(Hkv):
                for p in range(oc.next_page[0][h]):
                    assert np.array_equal(mine[h, p, :valid[h, p]], ref[0, h, p, :valid[h, p]]), (nm, h, p)
        for t, ref in ((cache.kmaster, oc.base_K_scale_master), (cache.vmaster, oc.base_V_scale_master)):
            n = oc.next_page[0][0]
            assert np.array_equal(t[0, :, 0, :n].cpu().numpy(), ref[0, :, :n])
    assert cache.next_slot[0].tolist() == [nk, nv]
    assert np.array_equal(cache.k_res[0, :nk].cpu().numpy(), oc.k_residual_buf[:nk])
    assert np.array_equal(cache.v_res[0, :nv].cpu().numpy(), oc.v_residual_buf[:nv])
    assert np.array_equal(cache.k_res_scale[0, :nk].cpu().numpy(), oc.k_residual_scale[:nk, 0])
    assert np.array_equal(cache.v_res_scale[0, :nv].cpu().numpy(), oc.v_residual_scale[:nv, 0])
    P = oc.next_page[0][0]
    for h in range(Hkv):
        for p in range(P):
            m = oc.meta_table[0][h][p]
            assert m is not None, (h, p)
            assert cache.k_slot[0, h, 0, p].tolist() == list(m.k_residual_slots), (h, p)
            assert cache.v_slot[0, h, 0, p].tolist() == list(m.v_residual_slots), (h, p)
    if base == "uniform":
        # the last decode-opened page reads back within INT3 error of its rows
        # (the reference's fixed-master encoding reads it back as zeros)
        kc, ks, vc, vs, lens = cache.read_base_concat(0, 0)
        nv_last = lens[-1]
        assert nv_last > 0 and len(lens) * 16 > T + 16
        kh = Q.dequantize(kc.cpu().numpy()[-nv_last:], ks.cpu().numpy()[-nv_last:], 32).astype(F32)
        rows = K[0, T + n_app - nv_last:T + n_app].astype(F32)
        gmax = np.abs(rows).reshape(nv_last, -1, 32).max(-1).repeat(32, -1)
        qmax = 2 ** (bits - 1) - 1
        assert np.abs(kh).max() > 0 and np.all(np.abs(kh - rows) <= gmax / qmax * 0.51 * 1.1 + 1e-3)
    # decode-filled pages hold slots now (the reference's fill store leaves
    # none); with the KIVI base a decode row is quantised alone, per channel
    # over one row, which is lossless for K (layer.py:1037-1075): no K slots
    if base == "uniform":
        assert any(s >= 0 for s in oc.meta_table[0][0][P - 2].k_residual_slots)
    out = care_kv.decode_attention(cache, 0, torch.from_numpy(Qh).cuda().unsqueeze(0))[0].cpu().numpy()
    ref = oracle_decode(oc, 0, Qh, k_mode="exact", kind="both", k_corr_scale=0.1, score_normalize=True,
                        kscore_live=True).astype(F32)
    err = np.abs(out.astype(F32) - ref)
    ulp = np.spacing(np.abs(ref).astype(F16)).astype(F32)
    assert np.all(err <= np.maximum(2e-3, ulp)), err.max()
    assert np.linalg.norm(out.astype(F32) - ref) <= 1e-2 * np.linalg.norm(ref)


# ------------------------------------------------------------------ router policies vs oracle
POLICY_CASES = [
    # policy, adaptive_score (rel, abs, min_keep) or None, live
    ("k_first", None, True),
    ("adaptive", None, True),
    ("k_first", None, False),
    ("adaptive", None, False),
    ("joint", (0.5, 0.0, 0), True),
    ("separate", (0.0, 1.5, 3), False),
    ("k_first", (0.8, 0.0, 2), True),
    ("adaptive", (0.3, 0.9, 0), False),
]


@pytest.mark.parametrize("D,Hq,Hkv,T", [(128, 8, 2, 700), (64, 16, 2, 400)], ids=["D128g4", "D64g8"])
@pytest.mark.parametrize("case", POLICY_CASES,
                         ids=[f"{c[0]}-{'as' if c[1] else 'fixed'}-{'live' if c[2] else 'proxy'}" for c in POLICY_CASES])
def test_decode_route_policies_vs_oracle(paper_env, case, D, Hq, Hkv, T):
    """The route-only policies (k_first, adaptive entropy split) and the
    adaptive_score thresholds (residual_router.py:305-410) on the GPU vs the
    oracle's route_selection, selections up to epsilon ties and outputs."""
    import care_kv
    pol, asc, live = case
    print(f"route policy case {case} D={D} Hq={Hq} Hkv={Hkv} T={T}", flush=True)
    paper_env.setenv("CAREKV_KSCORE_LIVE", "1" if live else "0")
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    eps = 1e-4 if live else 2e-3
    rng = np.random.default_rng(D + Hq + T + len(pol))
    K = rng.standard_normal((Hkv, T, D)).astype(F16)
    V = rng.standard_normal((Hkv, T, D)).astype(F16)
    K[:, :, rng.permutation(D)[:3]] *= F16(6.0)
    Qh = rng.standard_normal((Hq, D)).astype(F16)
    rel, ab, keep = asc if asc else (0.0, 0.0, 0)
    common = dict(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16, max_pages=T // 16 + 4,
                  base_bits=3, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                  read_budget_mode="adaptive_score" if asc else "absolute", read_abs_k=6, read_abs_v=6,
                  route_policy=pol, store_budget_mode="absolute", store_abs_k=2, store_abs_v=2,
                  read_relative_threshold=rel, read_absolute_threshold=ab, read_min_keep=keep)
    oc = OCache(OCfg(**common))
    for h in range(Hkv):
        write_pages_for_kv_head(oc, 0, h, K[h], V[h])
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0, **common)
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    cache.write_prefill(0, torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda())
    torch.cuda.synchronize()
    odiag = {}
    o_out = oracle_decode(oc, 0, Qh, k_mode="exact", kind="both", k_corr_scale=0.1, score_normalize=True,
                          kscore_live=live, diag=odiag)
    out, diag = care_kv.decode_attention(cache, 0, torch.from_numpy(Qh).cuda().unsqueeze(0), diag_cap=1024)
    out = out[0].cpu().numpy().astype(F32)
    diag = diag[0].cpu().numpy()
    grp = Hq // Hkv
    n_sel = n_tie = 0
    for h in range(Hkv):
        d = odiag[h]
        Kc, Vc = oracle_candidates(oc, 0, h, oc.next_page[0][h])
        ref_rows = oracle_selection(d, Kc, Vc)
        for j in range(grp):
            mine = set(decode_diag(diag[h * grp + j]))
            n_sel += len(ref_rows[j])
            n_tie += mine != ref_rows[j]
            for kind in (0, 1):  # the route policies and thresholds act per kind
                a_ = {c for c in mine if c[0] == kind}
                b_ = {c for c in ref_rows[j] if c[0] == kind}
                assert ties_explain(a_, b_, d, Kc, Vc, j, eps=eps), (h, j, kind, sorted(a_ ^ b_))
    assert n_sel > 0
    assert n_tie * 16 <= max(Hq, 16), n_tie  # at most 1 query row in 16 crosses a tie
    err = np.abs(out - o_out.astype(F32))
    assert err.max() <= 2e-3, err.max()


# ------------------------------------------------------------------ overflow status
def test_overflow_status_is_raised(paper_env):
    """The kernels flag what they cannot hold instead of dropping it
    silently: a page with more stored K slots than the decode records'
    capacity (forced from the host by lowering k_cap), and slot ids past a
    too-small slot arena.  With CAREKV_CHECK=1 the host reads the status word
    back and raises; a call without overflow after them passes (the status
    starts clear every call)."""
    import care_kv
    paper_env.setenv("CAREKV_CHECK", "1")
    rng = np.random.default_rng(7)
    D, Hq, Hkv, T = 64, 8, 2, 100
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16, max_pages=10,
                              base_bits=3, group_size=32, packed_base=True, scale_quant="int8",
                              store_budget_mode="absolute", store_abs_k=2, store_abs_v=2,
                              read_budget_mode="absolute", read_abs_k=4, read_abs_v=4, route_policy="joint",
                              read_budget_ratio=0.0)
    K = torch.from_numpy(rng.standard_normal((Hkv, T, D)).astype(F16)).cuda()
    V = torch.from_numpy(rng.standard_normal((Hkv, T, D)).astype(F16)).cuda()
    q = torch.from_numpy(rng.standard_normal((1, Hq, D)).astype(F16)).cuda()
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    cache.write_prefill(0, K, V)
    care_kv.decode_attention(cache, 0, q)  # no overflow
    cache.k_cap = 1  # two stored K slots per page, room for one
    with pytest.raises(care_kv.CarekvError, match="overflow"):
        care_kv.decode_attention(cache, 0, q)
    cache.k_cap = 2
    care_kv.decode_attention(cache, 0, q)  # the next call starts clear
    small = care_kv.CAREKVCache(cfg, device="cuda", n_slots=5)  # 7 pages x 2 kv heads x 2 slots do not fit
    with pytest.raises(care_kv.CarekvError, match="overflow"):
        small.write_prefill(0, K, V)


# ------------------------------------------------------------------ correction_impl=cached (the router path)
@pytest.mark.parametrize("name,Hq,D,k_mode,policy,store",
                         [("cached_gqa4_d64", 8, 64, "exact", "joint",
                           dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4)),
                          ("cached_mha_d128_linear", 2, 128, "linear", "separate",
                           dict(store_budget_mode="ratio", store_budget_ratio=0.03))])
def test_prefill_cached_matches_reference(paper_env, name, Hq, D, k_mode, policy, store):
    """CAREKVLayer.prefill in carekv_stored mode with correction_impl="cached",
    what CAREKVAdapter runs by default: the reference's per-(head, row)
    apply_slot_corrections over ResidualRouter.route (layer.py:573-640),
    whose golden was written with CAREKV_KSCORE_LIVE=0 (first case) and =1
    (second: the router ignores it).  The layer (identity projections) gives
    the reference output within the decode bar, with no warning."""
    import warnings

    import care_kv
    g = load_golden(f"prefill_{name}.npz")
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", k_mode)
    paper_env.setenv("CAREKV_KSCORE_LIVE", "1" if name.endswith("linear") else "0")
    paper_env.setenv("CAREKV_PREFILL_MODE", "carekv_stored")
    print(f"cached prefill golden {name}", flush=True)
    T, Hkv = int(g["T"]), 2
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                              max_pages=T // 16 + 4, base_bits=3, group_size=32, k_channel_group=32, v_token_block=4,
                              sketch_dim=32, packed_base=True, scale_quant="int8", read_budget_ratio=0.0,
                              read_budget_mode="absolute", read_abs_k=int(g["read_k"]), read_abs_v=int(g["read_v"]),
                              route_policy=policy, correction_impl="cached", **store)
    nq, nk = Hq * D, Hkv * D
    eye = torch.eye(nq + 2 * nk, dtype=torch.float16, device="cuda")
    lay = care_kv.CAREKVLayer(cfg, 0, eye[:nq].contiguous(), eye[nq:nq + nk].contiguous(),
                              eye[nq + nk:].contiguous(), eye[:nq, :nq].contiguous())
    Q, K, V = (torch.from_numpy(g[n]) for n in ("Q", "K", "V"))
    hidden = torch.cat([Q.reshape(T, -1), K.permute(1, 0, 2).reshape(T, -1), V.permute(1, 0, 2).reshape(T, -1)],
                       1).cuda()
    cache = care_kv.CAREKVCache(cfg, n_seq=1)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        out = lay.prefill(cache, hidden).float().cpu().numpy().reshape(T, Hq, D)
    compare_cache_to_golden(cache, g)
    ref = g["O"].astype(F32)
    err = np.abs(out - ref)
    assert np.all(err <= np.maximum(2e-3, np.spacing(np.abs(g["O"])).astype(F32))), err.max()
    assert np.abs(out - g["O_base"].astype(F32)).max() > 1e-2  # the correction did something
