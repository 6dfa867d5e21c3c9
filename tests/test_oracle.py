"""Pins the CPU oracle against the reference's golden vectors, the reference-held
activation arrays, closed forms and brute force.  CPU only."""
import math

import numpy as np
import pytest

from oracle import quant as Q
from oracle.attention import (decode_attention, exact_softmax_correction, prefill_stored,
                              query_aware_kscore_slot, softmax_rows,
                              vectorized_joint_correction)
from oracle.cache import OCache, OCfg
from oracle.store import decode_append, process_page, write_pages_for_kv_head

F16, F32 = np.float16, np.float32


# ------------------------------------------------------------ packing (closed form)
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_pack_roundtrip_and_bytes(bits):
    rng = np.random.default_rng(bits)
    lo, hi = -(2 ** (bits - 1)), 2 ** (bits - 1) - 1
    codes = rng.integers(lo, hi + 1, size=(37, 128)).astype(np.int8)
    p = Q.pack_codes_2d(codes, bits)
    assert p.shape == (37, Q.packed_row_bytes(128, bits))
    assert np.array_equal(Q.unpack_codes_2d(p, bits, 128), codes)
    flat = codes.ravel()[:101]
    p1 = {2: Q.pack_int2, 3: Q.pack_int3, 4: Q.pack_int4}[bits](flat)
    assert np.array_equal({2: Q.unpack_int2, 3: Q.unpack_int3, 4: Q.unpack_int4}[bits](p1, 101), flat)


def test_pack_bit_positions():
    # INT3: 8 codes -> 24-bit LE word sum((c_i & 7) << 3i)  (quantizer.py:304-324)
    c = np.array([[1, 2, 3, -1, -4, 0, -2, 3]], np.int8)
    word = sum((int(v) & 7) << (3 * i) for i, v in enumerate(c[0]))
    assert Q.pack_int3_2d(c).view(np.uint8).tolist() == [[word & 255, (word >> 8) & 255, word >> 16]]
    # INT4: low nibble = even index;  INT2: LSB first
    assert Q.pack_int4_2d(np.array([[3, -2]], np.int8)).view(np.uint8).tolist() == [[0x03 | (0x0E << 4)]]
    assert Q.pack_int2_2d(np.array([[1, -2, 0, -1]], np.int8)).view(np.uint8).tolist() == [[1 | (2 << 2) | (0 << 4) | (3 << 6)]]


def test_pack_4bit_roundtrip():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((16, 32)).astype(F32)
    p, s = Q.pack_4bit(x)
    r = Q.unpack_4bit(p, s, x.size).reshape(x.shape)
    assert p.shape == (256,)
    assert np.linalg.norm(r - x) / np.linalg.norm(x) < 0.3     # test_care_kv.py:69-74


# ------------------------------------------------------------ quantizer KAT
@pytest.mark.parametrize("layer", ["00", "21"])
def test_quantizer_fp32_against_reference_activations(golden, layer):
    """|dequant(quant(|x|))| vs the reference-held K_hat/V_hat (INT3, g=32, fp32).
    Cells where x/scale is an exact k+1/2 tie are exempt (the reference ran a
    different division)."""
    g = golden("activations_3d_slices.npz")
    for kv in ("k", "v"):
        x = g[f"l{layer}_{kv}_fp"]
        ref = g[f"l{layer}_{kv}_hat"]
        codes, scale = Q.quantize(x, 3, 32)
        xh = np.abs(Q.dequantize(codes, scale, 32))
        q = (x.reshape(x.shape[0], -1, 32) / scale[..., None]).reshape(x.shape)
        tie = np.abs(np.abs(q - np.floor(q)) - 0.5) < 1e-6
        diff = np.abs(xh - ref)
        assert diff[~tie].max() <= 1e-6
        assert tie.mean() < 1e-3


def test_quantizer_fp16_chain_matches_torch():
    """The fp16 rounding convention (fp32 op, round to fp16) equals torch's CPU
    half arithmetic; torch is the library the reference calls."""
    import torch
    x = (torch.randn(4096, 64) * 3).half()
    for bits in (2, 3, 4):
        qm = 2 ** (bits - 1) - 1
        m = x.reshape(-1, 2, 32).abs().amax(-1, keepdim=True).clamp(min=1e-8)
        sc = m / qm
        tq = (x.reshape(-1, 2, 32) / sc).round().clamp(-qm - 1, qm).to(torch.int8).reshape(x.shape)
        codes, scale = Q.quantize(x.numpy(), bits, 32)
        assert np.array_equal(codes, tq.numpy())
        assert np.array_equal(scale, sc[..., 0].numpy())


# ------------------------------------------------------------ store / cache goldens
def _cfg_from_store(tag, **kw):
    base = dict(num_layers=1, num_heads=2, num_kv_heads=2, head_dim=128, page_size=16, max_pages=8,
                base_bits=3, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32)
    if tag == "abs":
        base.update(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4)
    else:
        base.update(store_budget_mode="ratio", store_budget_ratio=0.03)
    base.update(kw)
    return OCfg(**base)


def _compare_cache(c: OCache, g, prefix="", err_ulp=1):
    L = 0
    H, P = c.valid_tokens.shape[1:]
    for nm, arr in (("K_codes", c.base_K_codes), ("V_codes", c.base_V_codes),
                    ("K_scale", c.base_K_scale), ("V_scale", c.base_V_scale),
                    ("K_master", c.base_K_scale_master), ("V_master", c.base_V_scale_master),
                    ("valid", c.valid_tokens)):
        ref = g[prefix + nm]
        mine = arr[L][:, :ref.shape[1]]
        valid = c.valid_tokens[L][:, :ref.shape[1]]
        if nm.endswith("codes") or nm.endswith("scale"):
            # padded rows of a partial page are never read; compare valid rows
            for h in range(ref.shape[0]):
                for p in range(ref.shape[1]):
                    n = int(valid[h, p])
                    assert np.array_equal(mine[h, p, :n], ref[h, p, :n]), (nm, h, p)
        else:
            assert np.array_equal(mine, ref), nm
    if prefix + "K_hat" in g:  # fp16 side buffer: every row, padded ones included (zeros)
        for nm, arr in (("K_hat", c.base_K_hat_fp16), ("V_hat", c.base_V_hat_fp16)):
            ref = g[prefix + nm]
            assert np.array_equal(arr[L][:, :ref.shape[1]].view(np.uint16), ref.view(np.uint16)), nm
    nk = g[prefix + "k_res"].shape[0]
    nv = g[prefix + "v_res"].shape[0]
    assert c.next_k_slot == nk and c.next_v_slot == nv
    assert np.array_equal(c.k_residual_buf[:nk], g[prefix + "k_res"])
    assert np.array_equal(c.k_residual_scale[:nk], g[prefix + "k_res_scale"])
    assert np.array_equal(c.v_residual_buf[:nv], g[prefix + "v_res"])
    assert np.array_equal(c.v_residual_scale[:nv], g[prefix + "v_res_scale"])
    for h in range(H):
        for p in range(g[prefix + "k_slots"].shape[1]):
            m = c.meta_table[L][h][p]
            if g[prefix + "k_slots"][h, p, 0] == -2:
                assert m is None
                continue
            assert m.k_residual_slots == g[prefix + "k_slots"][h, p].tolist()
            assert m.v_residual_slots == g[prefix + "v_slots"][h, p].tolist()
            for nm, ref in (("k_err", m.k_error_norm), ("v_err", m.v_error_norm), ("k_sketch", m.k_sketch)):
                a = ref.astype(F16).view(np.int16).astype(np.int32)
                b = g[prefix + nm][h, p].view(np.int16).astype(np.int32)
                assert np.abs(a - b).max() <= err_ulp, (nm, h, p)


@pytest.mark.parametrize("tag", ["abs", "ratio"])
def test_store_pages_golden(golden, tag):
    g = golden("store_d128.npz")
    c = OCache(_cfg_from_store(tag))
    for h in range(2):
        write_pages_for_kv_head(c, 0, h, g["K"][h], g["V"][h], token_start_abs=0, sink_tokens=4)
    _compare_cache(c, g, prefix=tag + "_")


def test_sketch_projection_fixture(golden):
    from oracle.store import sketch_proj
    import os
    ref = np.load(os.path.join(os.path.dirname(__file__), "golden", "sketch_proj_32x32.npy"))
    assert np.array_equal(sketch_proj(32, 32), ref)


def test_append_golden(golden):
    g = golden("append_d64.npz")
    cfg = OCfg(num_layers=1, num_heads=1, num_kv_heads=1, head_dim=64, page_size=16, max_pages=4,
               base_bits=3, group_size=32, store_budget_mode="absolute")
    c = OCache(cfg)
    X = g["X"]
    page = np.concatenate([X[:, :10], np.zeros((2, 6, 64), F16)], 1)
    Kc, Ks = Q.quantize(page[0], 3, 32)
    Vc, Vs = Q.quantize(page[1], 3, 32)
    p0 = c.alloc_page(0, 0)
    c.write_base(0, 0, p0, Kc, Ks, Vc, Vs, 10)
    for i in range(10, 16):
        kc, ks = Q.quantize(X[0, i:i + 1], 3, 32)
        vc, vs = Q.quantize(X[1, i:i + 1], 3, 32)
        c.append_to_page(0, 0, p0, kc[0], ks[0], vc[0], vs[0])
    p1 = c.alloc_page(0, 0)
    for i in range(16, 21):
        kc, ks = Q.quantize(X[0, i:i + 1], 3, 32)
        vc, vs = Q.quantize(X[1, i:i + 1], 3, 32)
        c.append_to_page(0, 0, p1, kc[0], ks[0], vc[0], vs[0])
    Kc2, Ks2, Vc2, Vs2, lens = c.read_base_concat(0, 0, [p0, p1])
    assert lens == g["read_lens"].tolist()
    for a, b in ((Kc2, "read_Kc"), (Ks2, "read_Ks"), (Vc2, "read_Vc"), (Vs2, "read_Vs")):
        assert np.array_equal(a, g[b]), b
    # decode-opened page: master 0 -> every scale reads back as 0 (reference behaviour)
    assert float(c.base_K_scale_master[0, 0, p1]) == 0.0 and np.all(Ks2[16:] == 0)


# ------------------------------------------------------------ decode goldens
from helpers import DECODE_CASES, PREFILL_CASES, build_oracle_prefill  # noqa: E402  (shared with the GPU tests)


def build_decode_case(g, name):
    """Rebuild the golden case's cache with the oracle (prefill pages + decode appends)."""
    spec = DECODE_CASES[name]
    T, n_app = int(g["T"]), int(g["n_append"])
    cfg = OCfg(num_layers=1, num_heads=spec["Hq"], num_kv_heads=spec["Hkv"], head_dim=spec["D"], page_size=16,
               max_pages=max(T // 16 + 4, 400), base_bits=spec.get("base_bits", 3), group_size=32,
               k_channel_group=32, v_token_block=4, sketch_dim=32, read_budget_mode="absolute",
               read_abs_k=int(g["read_k"]), read_abs_v=int(g["read_v"]), route_policy="joint",
               base_quantizer=spec.get("base_quantizer", "uniform"), **spec["store"])
    c = OCache(cfg)
    for h in range(spec["Hkv"]):
        write_pages_for_kv_head(c, 0, h, g["K"][h, :T], g["V"][h, :T], token_start_abs=0, sink_tokens=4)
    for t in range(T, T + n_app):
        decode_append(c, 0, g["K"][:, t], g["V"][:, t])
    return c, spec


def selection_matches(sel_a, sel_b, scores_r, budget, eps=1e-4):
    """Selections equal, except swaps between candidates whose normalised
    scores are within eps (relative) of the k-th largest score."""
    if np.array_equal(sel_a, sel_b):
        return True
    for q in range(sel_a.shape[0]):
        if np.array_equal(sel_a[q], sel_b[q]):
            continue
        s = scores_r[q]
        kth = np.sort(s)[::-1][budget - 1]
        diff = np.nonzero(sel_a[q] != sel_b[q])[0]
        if not np.all(np.abs(s[diff] - kth) <= eps * max(abs(kth), 1e-30)):
            return False
    return True


@pytest.mark.parametrize("name", list(DECODE_CASES))
def test_decode_golden(golden, name):
    g = golden(f"decode_{name}.npz")
    c, spec = build_decode_case(g, name)
    _compare_cache(c, g)
    diag = {}
    out = decode_attention(c, 0, g["Q"], k_mode=spec["k_mode"], kind="both", k_corr_scale=0.1,
                           score_normalize=True, kscore_live=spec.get("live", True), diag=diag)
    ref = g["O"].astype(F32)
    assert np.abs(out.astype(F32) - ref).max() <= 2e-3
    for h, d in diag.items():
        assert np.abs(d["O_base"] - g[f"h{h}_O_base"]).max() <= 1e-5
        if f"h{h}_sel_k" in g:
            sK, sV = d["score_K_r"], d["score_V_r"]
            merged = np.concatenate([sK, sV], 1)
            sel_ref = np.concatenate([g[f"h{h}_sel_k"], g[f"h{h}_sel_v"]], 1)
            sel_me = np.concatenate([d["sel_k"], d["sel_v"]], 1)
            mb = int(sel_ref[0].sum())
            assert selection_matches(sel_me, sel_ref, merged, mb)
            # the proxy's boundary term sums a_t / (s_top - s_t): near-top tokens
            # amplify the fp32 rounding of the logits (numpy vs torch order)
            np.testing.assert_allclose(d["score_K"], g[f"h{h}_score_K"], rtol=spec.get("score_rtol", 2e-5),
                                       atol=1e-12)
            np.testing.assert_allclose(d["score_V"], g[f"h{h}_score_V"], rtol=2e-5, atol=1e-12)
    if "decode_step_out" in g:
        # the reference decode_step itself (correction gated off by read_budget_ratio=0)
        base = decode_attention(c, 0, g["Q"], correction=False)
        assert np.abs(base.astype(F32) - g["decode_step_out"].astype(F32)).max() <= 2e-3


# ------------------------------------------------------------ prefill carekv_stored
@pytest.mark.parametrize("name", list(PREFILL_CASES))
def test_prefill_stored_golden(golden, name):
    """CAREKVLayer.prefill in carekv_stored mode with the vectorized
    correction (layer.py:538-557, 780-838): cache bytes, the base_quant
    output, the corrected output and the per-query selections."""
    g = golden(f"prefill_{name}.npz")
    c, spec, Kh, Vh = build_oracle_prefill(g, name)
    _compare_cache(c, g)
    Qh = g["Q"].transpose(1, 0, 2)
    base = prefill_stored(c, 0, Qh, Kh, Vh, correction=False)
    # torch's fp16 einsum and numpy's fp32 matmul sum in different orders:
    # up to 0.2% of the outputs land one fp16 rounding apart (where the sum
    # cancels, up to 1.2e-4 absolute on small outputs)
    ref = g["O_base"]
    err = np.abs(base.astype(F32) - ref.astype(F32))
    ulp = np.spacing(np.maximum(np.abs(ref), np.abs(base))).astype(F32)
    assert np.all(err <= np.maximum(ulp, 2.5e-4)) and np.mean(err > 0) < 5e-3, (err.max(), np.mean(err > 0))
    diag = {}
    out = prefill_stored(c, 0, Qh, Kh, Vh, k_mode=spec["k_mode"], kind="both", k_corr_scale=0.1,
                         score_normalize=True, kscore_live=True, diag=diag)
    err = np.abs(out.astype(F32) - g["O"].astype(F32))
    assert err.max() <= 1e-3, err.max()
    for h, d in diag.items():
        if f"h{h}_sel_k" in g:
            sK, sV = d["score_K_r"], d["score_V_r"]
            merged = np.concatenate([sK, sV], 1)
            # candidates of pages after a query's row score 0 (A = 0 there);
            # top-k picks among such ties arbitrarily and they change nothing
            pos = merged > 0
            sel_ref = np.concatenate([g[f"h{h}_sel_k"], g[f"h{h}_sel_v"]], 1) & pos
            sel_me = np.concatenate([d["sel_k"], d["sel_v"]], 1) & pos
            if spec["policy"] == "joint":
                mb = int(np.concatenate([g[f"h{h}_sel_k"], g[f"h{h}_sel_v"]], 1)[0].sum())
                assert selection_matches(sel_me, sel_ref, merged, mb)
            else:
                nk = sK.shape[1]
                for lo, hi, cap in ((0, nk, int(g["read_k"])), (nk, merged.shape[1], int(g["read_v"]))):
                    assert selection_matches(sel_me[:, lo:hi], sel_ref[:, lo:hi], merged[:, lo:hi],
                                             min(cap, hi - lo))
            # the weights are fp16 roundings of softmax values: where numpy's
            # and torch's fp32 softmax straddle a rounding point a weight
            # moves one fp16 ulp (2^-11 relative), and so does its score term
            for key in ("score_K", "score_V"):
                a, b = d[key], g[f"h{h}_{key}"]
                rel = np.abs(a - b) / np.maximum(np.abs(b), 1e-30)
                rel[(np.abs(a - b) <= 1e-12)] = 0.0
                assert rel.max() <= 1e-3 and np.mean(rel > 2e-5) < 1e-3, (key, rel.max(), np.mean(rel > 2e-5))


# ------------------------------------------------------------ reference test fixture grid
def test_reference_fixture_grid(golden):
    g = golden("ref_fixture_d32.npz")
    base = dict(num_layers=1, num_heads=3, num_kv_heads=1, head_dim=32, page_size=8, max_pages=4, base_bits=3,
                group_size=8, k_channel_group=16, v_token_block=4, store_budget_mode="absolute",
                read_budget_mode="absolute", store_abs_k=2, store_abs_v=2, read_abs_k=2, read_abs_v=2,
                sketch_dim=4, packed_base=False, scale_quant="none")
    from oracle.store import sketch_proj
    P = sketch_proj(16, 4)
    for pol in ("joint", "separate"):
        c = OCache(OCfg(route_policy=pol, **base))
        for p in range(4):
            Kc, Ks = Q.quantize(g["K"][p], 3, 8)
            Vc, Vs = Q.quantize(g["V"][p], 3, 8)
            pid = c.alloc_page(0, 0)
            c.write_base(0, 0, pid, Kc, Ks, Vc, Vs, 8)
            process_page(c, 0, 0, pid, g["K"][p], g["V"][p], Kc, Ks, Vc, Vs, token_start=p * 8, num_valid=8, P=P)
        if pol == "joint":
            assert np.array_equal(c.base_K_codes[0], g["cache_K_codes"])
            assert np.array_equal(c.k_residual_buf[:c.next_k_slot], g["cache_k_res"])
        pids = list(range(4))
        Kc, Ks, Vc, Vs, _ = c.read_base_concat(0, 0, pids)
        Kb = Q.dequantize(Kc, Ks, 8).astype(F32)
        Vb = Q.dequantize(Vc, Vs, 8).astype(F32)
        S = (g["Q"] @ Kb.T) / F32(math.sqrt(32))
        A = softmax_rows(S)
        O = A @ Vb
        for live in (0, 1):
            for mode in ("linear", "exact"):
                for kind in ("both", "k", "v"):
                    for norm in (False, True):
                        tag = f"{pol}_live{live}_{mode}_{kind}_n{int(norm)}"
                        d = {}
                        dl = vectorized_joint_correction(c, 0, 0, pids, g["Q"], S, A, Vb, O, kind=kind,
                                                         k_corr_scale=0.1, score_normalize=norm,
                                                         kscore_live=bool(live), k_mode=mode, sketch_P=P, diag=d)
                        np.testing.assert_allclose(dl, g[f"{tag}_delta"], atol=1e-5, err_msg=tag)
                        for key in ("sel_k", "sel_v"):
                            if f"{tag}_{key}" in g:
                                assert np.array_equal(d[key], g[f"{tag}_{key}"]), (tag, key)


# ------------------------------------------------------------ math pins
def test_exact_renorm_vs_fp64_bruteforce():
    """attention.py:96-118 against a direct fp64 softmax of (s + ds) (cf. the
    reference's tests/test_exact_k_correction.py:71-111)."""
    rng = np.random.default_rng(7)
    Qn, N, D = 3, 40, 16
    S = rng.standard_normal((Qn, N))
    A = softmax_rows(S.astype(F32))
    ds = np.zeros((Qn, N)); ds[:, 5:13] = rng.standard_normal((Qn, 8)) * 0.7
    V = rng.standard_normal((N, D)).astype(F32)
    RV = np.zeros((N, D), F32); RV[20:24] = rng.standard_normal((4, D)) * 0.1
    sel = np.zeros((Qn, N), bool); sel[:, 20:24] = True
    O = A @ V
    got = exact_softmax_correction(A, ds, V, O, RV, sel)
    a64 = np.exp(S + ds - (S + ds).max(1, keepdims=True)); a64 /= a64.sum(1, keepdims=True)
    ref = a64 @ V.astype(np.float64) + (a64 * sel) @ RV.astype(np.float64) - O
    assert np.abs(got - ref).max() < 1e-5
    # boundedness: ||O_new|| <= max ||V_t + RV_t||  (test_exact_k_correction.py:134-147)
    assert np.linalg.norm(O + got, axis=1).max() <= np.linalg.norm(V + RV, axis=1).max() + 1e-5


def test_kscore_closed_form():
    rng = np.random.default_rng(3)
    Qs, dK, A, Vs = (rng.standard_normal((2, 32)), rng.standard_normal((16, 32)),
                     rng.random((2, 16)) * 0.1, rng.standard_normal((16, 64)))
    got = query_aware_kscore_slot(Qs, dK, A, Vs, 128)
    ds = Qs @ dK.T / math.sqrt(128)
    ref = np.sqrt(((ds * A * (1 - A)) ** 2).sum(1)) * np.linalg.norm(Vs)
    np.testing.assert_allclose(got, ref, rtol=1e-5)


def test_read_zero_and_kind_v_invariants(golden):
    g = golden("decode_gqa4_d128.npz")
    c, spec = build_decode_case(g, "gqa4_d128")
    c.cfg.read_abs_k = c.cfg.read_abs_v = 0
    d0 = {}
    out0 = decode_attention(c, 0, g["Q"], correction=True, k_mode="exact", diag=d0)
    outb = decode_attention(c, 0, g["Q"], correction=False)
    assert np.array_equal(out0, outb)                       # READ=0 == base, bit-exact
    c.cfg.read_abs_k = c.cfg.read_abs_v = 8
    o_lin = decode_attention(c, 0, g["Q"], kind="v", k_mode="linear")
    o_ex = decode_attention(c, 0, g["Q"], kind="v", k_mode="exact")
    assert np.array_equal(o_lin, o_ex)                      # kind=v: exact == linear


# ---- prefill attention (layer.py:935-972)

def _prefill_inputs(Hq, Hkv, T, D, seed):
    rng = np.random.default_rng(seed)
    Qh = rng.standard_normal((Hq, T, D)).astype(np.float16)
    K = rng.standard_normal((Hkv, T, D)).astype(np.float16)
    V = rng.standard_normal((Hkv, T, D)).astype(np.float16)
    return Qh, K, V


def test_prefill_attention_vs_fp64_bruteforce():
    """Row-by-row float64 softmax attention (the textbook definition) on a
    tiny GQA input: the oracle differs only by its fp32 arithmetic and the
    fp16 cast of the weights and of O."""
    from oracle.attention import causal_attention_pure
    Hq, Hkv, T, D = 4, 2, 23, 32
    Qh, K, V = _prefill_inputs(Hq, Hkv, T, D, 5)
    O, lse = causal_attention_pure(Qh, K, V)
    for h in range(Hq):
        kv = h // (Hq // Hkv)
        for t in range(T):
            s = np.array([float(np.dot(Qh[h, t].astype(np.float64), K[kv, j].astype(np.float64))) / math.sqrt(D)
                          for j in range(t + 1)])
            w = np.exp(s - s.max())
            z = w.sum()
            o = (w / z) @ V[kv, :t + 1].astype(np.float64)
            np.testing.assert_allclose(O[h, t].astype(np.float64), o, atol=2e-3, rtol=2e-3)
            assert abs(lse[h, t] - (s.max() + math.log(z))) < 1e-4


def test_prefill_attention_causal_and_gqa_properties():
    from oracle.attention import causal_attention_pure
    Hq, Hkv, T, D = 4, 2, 40, 64
    Qh, K, V = _prefill_inputs(Hq, Hkv, T, D, 6)
    O, _ = causal_attention_pure(Qh, K, V)
    # the first query sees only token 0
    for h in range(Hq):
        assert np.array_equal(O[h, 0], V[h // 2, 0])
    # tokens after t do not change row t
    K2, V2 = K.copy(), V.copy()
    K2[:, 30:] = 7.0
    V2[:, 30:] = -3.0
    O2, _ = causal_attention_pure(Qh, K2, V2)
    assert np.array_equal(O[:, :30], O2[:, :30])
    # GQA: reading kv head h // 2 in place == repeat_interleave'd K/V
    Or, _ = causal_attention_pure(Qh, np.repeat(K, 2, axis=0), np.repeat(V, 2, axis=0))
    assert np.array_equal(O, Or)
    # row subsets agree with the full computation
    rows = [0, 17, 39]
    Os, _ = causal_attention_pure(Qh, K, V, rows=rows)
    assert np.array_equal(Os, O[:, rows])
    # without the mask the last row is unchanged and the first sees everything
    On, _ = causal_attention_pure(Qh, K, V, causal=False)
    assert np.array_equal(On[:, -1], O[:, -1])
    assert not np.array_equal(On[:, 0], O[:, 0])


# ------------------------------------------------------------ router policies
def test_route_selection_matches_reference(golden):
    """route_selection on the reference's raw candidate scores reproduces
    ResidualRouter.route's selections under every route_policy and the
    adaptive_score thresholds (fixture written by make_golden.py from
    residual_router.py:88-452), up to swaps inside a 1e-5 relative tie."""
    from oracle.attention import route_selection
    g = golden("route_d64.npz")
    variants = [("joint", None), ("separate", None), ("k_first", None), ("adaptive", None),
                ("joint", (0.5, 0.0, 0)), ("separate", (0.0, 1.5, 3)), ("k_first", (0.8, 0.0, 2)),
                ("adaptive", (0.3, 0.9, 0))]
    bk, bv = (int(x) for x in g["budgets"])
    n_checked = 0
    for h in range(2):
        sK, sV, A = g[f"h{h}_score_K"], g[f"h{h}_score_V"], g[f"h{h}_A"]
        kc = [tuple(x) for x in g[f"h{h}_kcand"].tolist()]
        vc = [tuple(x) for x in g[f"h{h}_vcand"].tolist()]
        for vi, (pol, asc) in enumerate(variants):
            for j in range(sK.shape[0]):
                rel, ab, keep = asc if asc else (0.0, 0.0, 0)
                selk, selv = route_selection(sK[j], sV[j], bk, bv, pol, "both", True, A_row=A[j],
                                             adaptive_score=asc is not None, rel_thr=rel, abs_thr=ab,
                                             min_keep=keep)
                mine_k = {kc[i] for i in np.nonzero(selk)[0]}
                mine_v = {vc[i] for i in np.nonzero(selv)[0]}
                ref_k = {tuple(x) for x in g[f"h{h}_v{vi}_q{j}_k"].tolist()}
                ref_v = {tuple(x) for x in g[f"h{h}_v{vi}_q{j}_v"].tolist()}
                for mine, ref, cand, s in ((mine_k, ref_k, kc, sK[j]), (mine_v, ref_v, vc, sV[j])):
                    if mine == ref:
                        continue
                    val = {c: float(s[i]) for i, c in enumerate(cand)}
                    kth = min(val[c] for c in ref) if ref else 0.0
                    assert all(abs(val[c] - kth) <= 1e-5 * max(abs(kth), 1e-30) for c in mine ^ ref), \
                        (h, pol, asc, j, sorted(mine ^ ref))
                n_checked += 1
    assert n_checked == 2 * len(variants) * 4


def test_streaming_fill_store_gives_decode_pages_slots():
    """decode_append(streaming=True) (no reference counterpart): a page the
    appends fill is stored from its true rows against its own codes, so it
    gets residual slots, and those residuals are true minus read-back base;
    the reference's fill store (streaming=False) gives the same page none."""
    rng = np.random.default_rng(3)
    D, H, T, n = 64, 1, 20, 30
    K = rng.standard_normal((H, T + n, D)).astype(F16)
    V = rng.standard_normal((H, T + n, D)).astype(F16)
    kw = dict(num_layers=1, num_heads=2, num_kv_heads=H, head_dim=D, page_size=16, max_pages=8, base_bits=3,
              group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32, store_budget_mode="absolute",
              store_abs_k=2, store_abs_v=4)
    slots = {}
    for streaming in (False, True):
        c = OCache(OCfg(**kw))
        write_pages_for_kv_head(c, 0, 0, K[0, :T], V[0, :T])
        for t in range(T, T + n):
            decode_append(c, 0, K[:, t], V[:, t], streaming=streaming)
        slots[streaming] = [c.meta_table[0][0][p].k_residual_slots for p in (1, 2)]
    assert all(s < 0 for row in slots[False] for s in row)
    assert all(sum(s >= 0 for s in row) == 2 for row in slots[True])


def test_prefill_stored_read_zero_is_base(golden):
    """READ = 0 in carekv_stored mode is the base_quant output bit for bit
    (layer.py:810-823), and the causal base of the first rows does not see
    the later tokens: truncating the prompt leaves those rows unchanged up
    to fp32 summation order.  (The correction of a row
    does depend on later pages: their candidates count in the normalisation
    and the budgets.)"""
    g = golden("prefill_gqa8_d64.npz")
    c, spec, Kh, Vh = build_oracle_prefill(g, "gqa8_d64")
    c.cfg.read_abs_k = c.cfg.read_abs_v = 0
    Qh = g["Q"].transpose(1, 0, 2)
    corr = prefill_stored(c, 0, Qh, Kh, Vh, k_mode="exact", kind="both", k_corr_scale=0.1, score_normalize=True,
                          kscore_live=True)
    base = prefill_stored(c, 0, Qh, Kh, Vh, correction=False)
    assert np.array_equal(corr.view(np.uint16), base.view(np.uint16))
    T = Qh.shape[1]
    short = prefill_stored(c, 0, Qh[:, :T // 2], Kh[:, :T // 2], Vh[:, :T // 2], correction=False)
    ref = base[:T // 2]
    err = np.abs(short.astype(F32) - ref.astype(F32))
    # (where the sum cancels, a few small outputs move up to 2.4e-4)
    assert np.all(err <= np.maximum(np.spacing(np.maximum(np.abs(ref), np.abs(short))).astype(F32), 2.5e-4))


# ------------------------------------------------------------ the router path (correction_impl=cached, decode_step)
CACHED_PREFILL_CASES = {
    "cached_gqa4_d64": dict(Hq=8, Hkv=2, D=64, store=dict(store_budget_mode="absolute", store_abs_k=2,
                                                           store_abs_v=4), k_mode="exact", policy="joint"),
    "cached_mha_d128_linear": dict(Hq=2, Hkv=2, D=128, store=dict(store_budget_mode="ratio", store_budget_ratio=0.03),
                                   k_mode="linear", policy="separate"),
}


def _oracle_prompt(g, spec, T):
    oc = OCache(OCfg(num_layers=1, num_heads=spec["Hq"], num_kv_heads=spec["Hkv"], head_dim=spec["D"], page_size=16,
                     max_pages=T // 16 + 4, base_bits=3, group_size=32, k_channel_group=32, v_token_block=4,
                     sketch_dim=32, read_budget_mode="absolute", read_abs_k=int(g["read_k"]),
                     read_abs_v=int(g["read_v"]), route_policy=spec["policy"], **spec["store"]))
    hats = [write_pages_for_kv_head(oc, 0, h, g["K"][h, :T], g["V"][h, :T]) for h in range(spec["Hkv"])]
    return oc, np.stack([a for a, _ in hats]), np.stack([b for _, b in hats])


@pytest.mark.parametrize("name", list(CACHED_PREFILL_CASES))
def test_prefill_cached_golden(golden, name):
    """CAREKVLayer.prefill in carekv_stored mode with correction_impl="cached"
    (per-(head, row) apply_slot_corrections over ResidualRouter.route,
    layer.py:573-640): the oracle's batched correction with the router's
    sketch-proxy K score gives the reference output within 1e-3; the
    query-aware K score does not (the cached path reads no KSCORE_LIVE, and
    the second golden was written with CAREKV_KSCORE_LIVE=1)."""
    g = golden(f"prefill_{name}.npz")
    spec = CACHED_PREFILL_CASES[name]
    T = int(g["T"])
    oc, Kh, Vh = _oracle_prompt(g, spec, T)
    _compare_cache(oc, g)
    Qh = g["Q"].transpose(1, 0, 2)
    kw = dict(k_mode=spec["k_mode"], kind="both", k_corr_scale=0.1, score_normalize=True)
    proxy = prefill_stored(oc, 0, Qh, Kh, Vh, kscore_live=False, **kw)
    err = np.abs(proxy.astype(F32) - g["O"].astype(F32))
    assert err.max() <= 1e-3, err.max()
    live = prefill_stored(oc, 0, Qh, Kh, Vh, kscore_live=True, **kw)
    assert np.abs(live.astype(F32) - g["O"].astype(F32)).max() > 1e-2


@pytest.mark.parametrize("name,Hq,D,k_mode,policy",
                         [("gqa4_d128", 8, 128, "exact", "joint"), ("gqa8_d64_linear", 16, 64, "linear", "separate")])
def test_decode_step_corrected_golden(golden, name, Hq, D, k_mode, policy):
    """The reference's decode_step with its correction gate open
    (read_budget_ratio > 0, attention.py:1025): apply_slot_corrections over
    ResidualRouter.route per query head.  The oracle's decode_append (store
    on fill with K_orig = K_hat, zero master on the decode-opened page) and
    decode_attention with the sketch-proxy selector give every step's output
    within the decode bar."""
    g = golden(f"decode_step_{name}.npz")
    T, n = int(g["T"]), int(g["n_append"])
    store = (dict(store_budget_mode="absolute", store_abs_k=2, store_abs_v=4) if name == "gqa4_d128"
             else dict(store_budget_mode="ratio", store_budget_ratio=0.03))
    spec = dict(Hq=Hq, Hkv=2, D=D, policy=policy, store=store)
    oc = OCache(OCfg(num_layers=1, num_heads=Hq, num_kv_heads=2, head_dim=D, page_size=16, max_pages=(T + n) // 16 + 4,
                     base_bits=3, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                     read_budget_mode="absolute", read_abs_k=int(g["read_k"]), read_abs_v=int(g["read_v"]),
                     route_policy=policy, **store))
    for h in range(2):
        write_pages_for_kv_head(oc, 0, h, g["K"][h, :T], g["V"][h, :T])
    for i, t in enumerate(range(T, T + n)):
        decode_append(oc, 0, g["K"][:, t], g["V"][:, t])
        o = decode_attention(oc, 0, g["Qall"][i], k_mode=k_mode, kind="both", k_corr_scale=0.1,
                             score_normalize=True, kscore_live=False)
        ref = g["outs"][i]
        err = np.abs(o.astype(F32) - ref.astype(F32))
        assert np.all(err <= np.maximum(2e-3, np.spacing(np.abs(ref)).astype(F32))), (i, err.max())
    _compare_cache(oc, g)
    del spec


def test_streaming_fill_store_residuals_are_true_minus_base():
    """decode_append(streaming=True): the K and V residual slots of a page the
    decode appends fill hold pack_4bit of (true rows - the page's own
    dequantised rows), K per 32-channel group over the page's 16 rows and V
    per 4-row block, and its error norms are those residuals' row-norm
    means."""
    rng = np.random.default_rng(5)
    D, T, n = 64, 20, 30
    K = rng.standard_normal((1, T + n, D)).astype(F16)
    V = rng.standard_normal((1, T + n, D)).astype(F16)
    K[:, :, 7] *= F16(6.0)
    c = OCache(OCfg(num_layers=1, num_heads=2, num_kv_heads=1, head_dim=D, page_size=16, max_pages=8, base_bits=3,
                    group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32, store_budget_mode="absolute",
                    store_abs_k=2, store_abs_v=4))
    write_pages_for_kv_head(c, 0, 0, K[0, :T], V[0, :T])
    for t in range(T, T + n):
        decode_append(c, 0, K[:, t], V[:, t], streaming=True)
    for p in (1, 2):  # the prompt's partial page refilled by decode, a decode-opened page
        m = c.meta_table[0][0][p]
        rows = slice(p * 16, p * 16 + 16)
        for nm, X, codes, which in (("K", K[0, rows], c.base_K_codes, "K"), ("V", V[0, rows], c.base_V_codes, "V")):
            Xh = Q.dequantize(c.unpack_rows(codes[0, 0, p]), c.page_scales(0, 0, p, which), 32).astype(F16)
            R = (X.astype(F16) - Xh).astype(F16).astype(F32)
            if nm == "K":
                for cg, slot in enumerate(m.k_residual_slots):
                    if slot < 0:
                        continue
                    blk = R[:, cg * 32:(cg + 1) * 32]
                    packed, scale = Q.pack_4bit(blk.ravel())
                    assert np.array_equal(c.k_residual_buf[slot], packed), (p, cg)
                    assert c.k_residual_scale[slot, 0] == scale, (p, cg)
                    want = F16(np.mean(np.sqrt((blk.astype(F32) ** 2).sum(1))))
                    assert abs(float(m.k_error_norm[cg]) - float(want)) <= float(np.spacing(want)), (p, cg)
            else:
                for vb, slot in enumerate(m.v_residual_slots):
                    if slot < 0:
                        continue
                    blk = R[vb * 4:(vb + 1) * 4]
                    packed, scale = Q.pack_4bit(blk.ravel())
                    assert np.array_equal(c.v_residual_buf[slot], packed), (p, vb)
                    assert c.v_residual_scale[slot, 0] == scale, (p, vb)
        assert sum(s >= 0 for s in m.k_residual_slots) == 2 and sum(s >= 0 for s in m.v_residual_slots) == 4


def test_reencoding_append_matches_write_base():
    """decode_append(rescale=True) (the compat=False append; no reference
    counterpart): after 16 appends a decode-opened page holds exactly the
    codes, int8 scale codes and master that write_base gives those 16 rows
    (cache.py:592-654); the prompt's partial page, which holds stored slots,
    keeps the reference's fixed-master encoding (its prefill scale codes and
    master); an open page reads back within INT3 quantisation error of its
    rows (the reference's encoding reads a decode-opened page back as
    zeros)."""
    rng = np.random.default_rng(11)
    D, T, n = 64, 20, 30
    K = (rng.standard_normal((1, T + n, D)) * np.exp(rng.standard_normal((1, 1, D)))).astype(F16)
    V = rng.standard_normal((1, T + n, D)).astype(F16)
    kw = dict(num_layers=1, num_heads=2, num_kv_heads=1, head_dim=D, page_size=16, max_pages=8, base_bits=3,
              group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32, store_budget_mode="absolute",
              store_abs_k=1, store_abs_v=1)
    c = OCache(OCfg(**kw))
    ref = OCache(OCfg(**kw))
    write_pages_for_kv_head(c, 0, 0, K[0, :T], V[0, :T])
    for t in range(T, T + n):
        decode_append(c, 0, K[:, t], V[:, t], rescale=True)
        if t == T + 20:  # page 2 (tokens 32..47) is open with 9 rows: check its first 5
            p, nv = 2, 5
            rows = slice(32, 32 + nv)
            for X, codes, which in ((K, c.base_K_codes, "K"), (V, c.base_V_codes, "V")):
                got = Q.dequantize(c.unpack_rows(codes[0, 0, p])[:nv], c.page_scales(0, 0, p, which)[:nv], 32)
                want = Q.dequantize(*Q.quantize(X[0, rows], 3, 32), 32)  # INT3 with fp16 scales
                err = np.abs(got.astype(F32) - X[0, rows].astype(F32))
                bound = np.abs(X[0, rows].astype(F32)).reshape(nv, -1, 32).max(-1).repeat(32, -1) / 3 * 0.51 + 1e-3
                assert np.all(err <= bound * 1.1) and np.abs(got).max() > 0, which
                assert np.abs(got.astype(F32) - want.astype(F32)).max() <= 0.05 * np.abs(want).max(), which
    # page 1 (prompt rows 16..19, then appends) holds slots: not re-encoded
    pre = OCache(OCfg(**kw))
    write_pages_for_kv_head(pre, 0, 0, K[0, :T], V[0, :T])
    assert any(x >= 0 for x in pre.meta_table[0][0][1].k_residual_slots)
    assert np.array_equal(c.base_K_scale[0, 0, 1, :4], pre.base_K_scale[0, 0, 1, :4])
    assert c.base_K_scale_master[0, 0, 1] == pre.base_K_scale_master[0, 0, 1]
    assert c.base_V_scale_master[0, 0, 1] == pre.base_V_scale_master[0, 0, 1]
    for p in (2,):  # page 2: decode-opened
        rows = slice(p * 16, p * 16 + 16)
        pid = ref.alloc_page(0, 0)
        Kc, Ks = Q.quantize(K[0, rows], 3, 32)
        Vc, Vs = Q.quantize(V[0, rows], 3, 32)
        ref.write_base(0, 0, pid, Kc, Ks, Vc, Vs, num_valid=16)
        for a, b in ((c.base_K_codes, ref.base_K_codes), (c.base_V_codes, ref.base_V_codes),
                     (c.base_K_scale, ref.base_K_scale), (c.base_V_scale, ref.base_V_scale)):
            assert np.array_equal(a[0, 0, p], b[0, 0, pid]), p
        assert c.base_K_scale_master[0, 0, p] == ref.base_K_scale_master[0, 0, pid]
        assert c.base_V_scale_master[0, 0, p] == ref.base_V_scale_master[0, 0, pid]
    # the reference's encoding: a decode-opened page reads back as zeros
    z = OCache(OCfg(**kw))
    write_pages_for_kv_head(z, 0, 0, K[0, :T], V[0, :T])
    for t in range(T, T + 20):
        decode_append(z, 0, K[:, t], V[:, t])
    assert np.all(Q.dequantize(z.unpack_rows(z.base_K_codes[0, 0, 2])[:4], z.page_scales(0, 0, 2, "K")[:4], 32) == 0)


def test_reencoding_keeps_slot_pages_and_fill_reuses_their_slots():
    """The compat=False decode append (streaming + rescale, no reference
    counterpart) on a prompt whose partial last page holds stored slots, when
    the appended rows are 16x larger than the prompt's: the page keeps its
    prefill encoding (the reference's fixed master), so each of its prompt
    rows still reads back as K_hat with K_hat + its K slot residual within
    the 4-bit residual error of the true row (re-encoding against the raised
    master would move K_hat away from the residual's base: 0.49 of the
    residual range here against 0.09); when the page fills, its new slots
    reuse the prefill's slot ids, so the page takes no new K id."""
    rng = np.random.default_rng(21)
    D, T, n = 64, 20, 12
    K = rng.standard_normal((1, T + n, D)).astype(F16)
    V = rng.standard_normal((1, T + n, D)).astype(F16)
    K[:, T:] *= F16(16.0)
    V[:, T:] *= F16(16.0)
    kw = dict(num_layers=1, num_heads=2, num_kv_heads=1, head_dim=D, page_size=16, max_pages=8, base_bits=3,
              group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32, store_budget_mode="absolute",
              store_abs_k=2, store_abs_v=1)
    c = OCache(OCfg(**kw))
    write_pages_for_kv_head(c, 0, 0, K[0, :T], V[0, :T])
    m0 = c.meta_table[0][0][1]
    k_ids, v_ids = list(m0.k_residual_slots), list(m0.v_residual_slots)
    nk0, nv0 = c.next_k_slot, c.next_v_slot
    assert sorted(k_ids) == [nk0 - 2, nk0 - 1] and sum(x >= 0 for x in v_ids) == 1
    km0, sc0 = c.base_K_scale_master[0, 0, 1], c.base_K_scale[0, 0, 1, :4].copy()

    def corrected_err(cache):
        Kh = Q.dequantize(cache.unpack_rows(cache.base_K_codes[0, 0, 1])[:4], cache.page_scales(0, 0, 1, "K")[:4], 32)
        worst = 0.0
        for cg, slot in enumerate(m0.k_residual_slots):
            R = Q.unpack_4bit(cache.k_residual_buf[slot], cache.k_residual_scale[slot, 0], 16 * 32).reshape(16, 32)
            cols = slice(cg * 32, cg * 32 + 32)
            rel = np.abs(Kh[:, cols].astype(F32) + R[:4] - K[0, 16:20, cols].astype(F32))
            worst = max(worst, float(rel.max()) / float(np.abs(R).max() + 1e-6))
        return worst

    for t in range(T, T + 5):  # the page still open
        decode_append(c, 0, K[:, t], V[:, t], streaming=True, rescale=True)
    assert c.base_K_scale_master[0, 0, 1] == km0 and np.array_equal(c.base_K_scale[0, 0, 1, :4], sc0)
    # 4-bit residual rounding (1/14 of the range) plus the int8 scale-code rounding of the prompt
    assert corrected_err(c) <= 0.2, corrected_err(c)
    for t in range(T + 5, T + n):  # fills the page
        decode_append(c, 0, K[:, t], V[:, t], streaming=True, rescale=True)
    m1 = c.meta_table[0][0][1]
    assert sorted(x for x in m1.k_residual_slots if x >= 0) == sorted(k_ids)
    used_v = sorted(x for x in m1.v_residual_slots if x >= 0)
    assert used_v[:1] == sorted(x for x in v_ids if x >= 0)  # the prefill's V id first, then new ones
    assert c.next_k_slot == nk0 and c.next_v_slot == nv0 + len(used_v) - 1
    # a page without slots is re-encoded by the same appends
    z = OCache(OCfg(**{**kw, "store_abs_k": 0, "store_abs_v": 0}))
    write_pages_for_kv_head(z, 0, 0, K[0, :T], V[0, :T])
    before = z.page_scales(0, 0, 1, "K")[:4].copy()
    for t in range(T, T + 5):
        decode_append(z, 0, K[:, t], V[:, t], streaming=True, rescale=True)
    assert not np.array_equal(z.page_scales(0, 0, 1, "K")[:4], before)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_kivi_codes_dequantise_to_kivi_qdq(bits):
    """The packed KIVI form (no reference counterpart) against the side
    buffer the reference keeps: half(code * scale) equals kivi_qdq (pinned
    by the KIVI decode goldens' K_hat / V_hat) up to the sign of zero, NaN
    where it is NaN (an all-zero K channel, an all-zero V row, a zero
    component of a one-row K); the codes lie in [-2^(b-1), 2^(b-1) - 1]."""
    rng = np.random.default_rng(bits)
    X = (rng.standard_normal((3, 70, 128)) * np.exp(rng.standard_normal((1, 1, 128)))).astype(np.float16)
    X[1, :, 5] = 0
    X[2, 9, :] = 0
    X[0, 3, 11] = 0
    qm = 2 ** (bits - 1)
    cases = [(X, True), (X, False), (X[0, 3:4], True)]
    for x, per_channel in cases:
        codes, scale = Q.kivi_codes(x, bits, per_channel)
        assert codes.min() >= -qm and codes.max() <= qm - 1
        got = (codes.astype(np.float32) * scale.astype(np.float32)).astype(np.float16)
        ref = Q.kivi_qdq(x, bits, per_channel)
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan), per_channel
        assert np.array_equal(got[~nan], ref[~nan]), per_channel    # +0 == -0
    # the NaNs come from the all-zero channel / row and the one-row zero, nowhere else
    assert np.isnan(Q.kivi_qdq(X, bits, True)[1, :, 5]).all()
    assert np.isnan(Q.kivi_qdq(X, bits, False)[2, 9]).all()
    assert np.isnan(Q.kivi_qdq(X[0, 3:4], bits, True)[0, 11])


@pytest.mark.parametrize("name", ["eval_gqa4_d64", "eval_mha_d128_k", "eval_gqa2_d128_v"])
def test_prefill_eval_golden(golden, name):
    """CAREKVLayer.prefill in carekv_eval mode (layer.py:792-806, 363-456)
    against the reference's output: the token-level top-k correction from
    the in-memory residuals over the causal fp16 base.  The base differs
    from torch's fp16 einsum by fp32 summation order (one fp16 rounding on
    a fraction of the outputs), which can also move a score by that much."""
    from helpers import EVAL_CASES, eval_hats, eval_knobs
    from oracle.attention import prefill_eval
    g = golden(f"prefill_{name}.npz")
    spec = EVAL_CASES[name]
    Kh, Vh = eval_hats(g, spec)
    T = int(g["T"])
    out = prefill_eval(g["Q"].transpose(1, 0, 2), g["K"][:, :T], g["V"][:, :T], Kh, Vh, **eval_knobs(g))
    ref = g["O"]
    err = np.abs(out.astype(F32) - ref.astype(F32))
    ulp = np.spacing(np.maximum(np.abs(ref), np.abs(out)).astype(F16)).astype(F32)
    assert np.all(err <= np.maximum(2 * ulp, 5e-4)), (err.max(), np.unravel_index(err.argmax(), err.shape))
    assert np.mean(err > 0) < 2e-2, np.mean(err > 0)
    # the correction changed the output (it is not the base)
    from oracle.attention import causal_attention_pure
    base, _ = causal_attention_pure(g["Q"].transpose(1, 0, 2), Kh, Vh)
    assert np.abs(base.transpose(1, 0, 2).astype(F32) - ref.astype(F32)).max() > 1e-2


@pytest.mark.parametrize("knobs", [dict(ratio=0.05, kind="both", normalize=True), dict(ratio=0.1, kind="k"),
                                   dict(ratio=0.03, kind="v", min_residuals=2)], ids=["both", "k", "v"])
def test_prefill_eval_rows_equal_full(knobs):
    """prefill_eval(rows=...) (the long-prompt form, each row's weights
    from that row alone) gives the full evaluation's selections on those
    rows, its scores up to the fp32 order of a one-row product (1e-5 of
    the row's largest score), outputs
    within one fp16 ulp (equal here), and leaves the other rows at the base."""
    from oracle.attention import causal_attention_pure, prefill_eval
    rng = np.random.default_rng(3)
    Hq, Hkv, D, T = 4, 2, 64, 150
    K = rng.standard_normal((Hkv, T, D)).astype(F16)
    V = rng.standard_normal((Hkv, T, D)).astype(F16)
    Qh = (rng.standard_normal((Hq, T, D)) * 0.7).astype(F16)
    Kh = Q.dequantize(*Q.quantize(K, 2, 32), 32)
    Vh = Q.dequantize(*Q.quantize(V, 2, 32), 32)
    O = causal_attention_pure(Qh, Kh, Vh)[0]
    d1, d2 = {}, {}
    full = prefill_eval(Qh, K, V, Kh, Vh, o_base=O, diag=d1, **knobs)
    rows = [0, 17, 63, 149]
    part = prefill_eval(Qh, K, V, Kh, Vh, o_base=O, diag=d2, rows=rows, **knobs)
    assert sorted(d2) == sorted((h, t) for h in range(Hq) for t in rows)
    for key, (idx, sc) in d2.items():
        assert np.array_equal(idx, d1[key][0]), key
        assert np.abs(sc - d1[key][1]).max() <= 1e-5 * np.abs(d1[key][1]).max(), key
    ulp = np.spacing(np.abs(full[rows]).astype(F16)).astype(F32)
    assert np.all(np.abs(part[rows].astype(F32) - full[rows].astype(F32)) <= ulp)
    others = [t for t in range(T) if t not in rows]
    assert np.array_equal(part[others], O.transpose(1, 0, 2)[others])


def test_pack_8bit_closed_form():
    """pack_8bit / unpack_8bit and the 8-bit branches of pack_residual /
    unpack_residual (residual_store.py:149-176): s = max|x| / 127 in fp32,
    codes = clamp(round-half-even(x / s), -128, 127) as int8, stored scale
    half(s), unpack = code * float(half(s)).  Checked on values whose codes
    the closed form fixes (s = 1 exactly; ties to even), on the all-zero
    block (1e-8 floor: every code 0, the fp16 scale underflows to 0), and on
    random blocks through the round-trip bound |x - x'| <= s / 2 + the fp16
    scale's rounding."""
    x = np.array([127, -127, 63.5, 62.5, 0.4, -0.6, -1.5, 0], F32)
    codes, scale = Q.pack_8bit(x)
    assert codes.dtype == np.int8 and scale.dtype == F16 and float(scale) == 1.0
    assert codes.tolist() == [127, -127, 64, 62, 0, -1, -2, 0]
    assert np.array_equal(Q.unpack_8bit(codes, scale, 8), codes.astype(F32))
    for bits, pk, uk in ((8, Q.pack_8bit, Q.unpack_8bit), (4, Q.pack_4bit, Q.unpack_4bit)):
        a, sa = Q.pack_residual(x, bits)
        b, sb = pk(x)
        assert np.array_equal(a, b) and sa == sb, bits
        assert np.array_equal(Q.unpack_residual(a, sa, 8, bits), uk(b, sb, 8)), bits
    z, sz = Q.pack_8bit(np.zeros((4, 64), F32))
    assert z.shape == (256,) and not z.any() and float(sz) == 0.0
    rng = np.random.default_rng(8)
    for _ in range(20):
        blk = (rng.standard_normal((4, 64)) * np.exp(rng.standard_normal())).astype(F32)
        c, s = Q.pack_8bit(blk)
        s32 = F32(F32(np.abs(blk).max()) / F32(127.0))
        assert np.array_equal(c, np.clip(np.rint(blk / s32), -128, 127).astype(np.int8).ravel())
        back = Q.unpack_8bit(c, s, blk.size).reshape(blk.shape)
        assert np.all(np.abs(back - blk) <= s32 / 2 + 127 * abs(float(s) - float(s32)) + 1e-6)


def test_layer_budget_multiplier_closed_form():
    """layer_budget_multiplier (cache.py:166-202) in the oracle and in the
    product (care_kv.config): uniform and one layer give 1; u_shaped gives
    w_l = 0.5 + 1.5 |2 l / (L - 1) - 1| over its mean (L = 3: 4/3, 1/3, 4/3;
    L = 5: w = 2, 1.25, 0.5, 1.25, 2 over 1.4), whose mean is 1;
    sensitivity gives s_l / mean(s), or 1 when the mean is not positive;
    layer_head_impact is uniform-equivalent."""
    from oracle.cache import layer_budget_multiplier as olbm
    from care_kv.config import CacheConfig, layer_budget_multiplier as plbm

    def both(L, policy, sens=None):
        oc = OCfg(num_layers=L, num_heads=4, num_kv_heads=2, head_dim=64, budget_policy=policy,
                  layer_sensitivity=sens)
        pc = CacheConfig(num_layers=L, num_heads=4, num_kv_heads=2, head_dim=64, budget_policy=policy,
                         layer_sensitivity=sens)
        o = [olbm(oc, l) for l in range(L)]
        p = [plbm(pc, l) for l in range(L)]
        assert np.allclose(o, p, rtol=0, atol=1e-15), (L, policy, o, p)
        return o

    assert both(4, "uniform") == [1.0] * 4
    assert both(1, "u_shaped") == [1.0] and both(1, "sensitivity", [3.0]) == [1.0]
    assert np.allclose(both(3, "u_shaped"), [4 / 3, 1 / 3, 4 / 3], rtol=1e-14)
    assert np.allclose(both(5, "u_shaped"), np.array([2, 1.25, 0.5, 1.25, 2]) / 1.4, rtol=1e-14)
    assert abs(np.mean(both(22, "u_shaped")) - 1.0) < 1e-12
    assert np.allclose(both(3, "sensitivity", [1.0, 2.0, 3.0]), [0.5, 1.0, 1.5], rtol=1e-14)
    assert both(3, "sensitivity", [0.0, 0.0, 0.0]) == [1.0] * 3
    assert both(3, "sensitivity", [1.0, -2.0, 0.5]) == [1.0] * 3
    assert both(3, "layer_head_impact") == [1.0] * 3
