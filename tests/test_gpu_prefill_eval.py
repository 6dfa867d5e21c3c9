"""Prefill in carekv_eval mode on the GPU (``carekv_prefill_eval``):
``_apply_sparse_prefill_correction_eval`` (layer.py:363-456) over the causal
base, as ``CAREKVLayer.prefill`` calls it (layer.py:792-806).

Bars.  The correction is held to the oracle (``prefill_eval``) over the
same base output o (the device's ``carekv_prefill_attn``, itself held to
the oracle's causal attention within 2e-3 in tests/test_gpu_prefill.py).
The selections equal the oracle's, ties to the lower index, except where
the two score sets tie to within 1e-5 of the row's largest score (the base
weights are both the fp32 softmax cast to fp16, but exp and the sum differ
in their last fp32 bits).  The oracle is then run with the device's
selections: every output is within max(2 fp16 ulps, 5e-4) of it, plus,
on at most 2% of the (head, row)s, one fp16 rounding of each selected
weight a_j carried through (sum over the selected j of
2^-11 (|r_v,j| + 2 k_corr |V_hat_j - o|)): the case of an a_j on an fp16
rounding boundary.  Against the reference's golden output, on the rows
whose selection equals the oracle's top-k: the output differs by at most
the device base's own difference from the reference's base (the oracle's
causal attention) plus one fp16 ulp of the output plus that same
allowance, and by relative L2 1e-2."""
import numpy as np
import pytest
import torch

from helpers import EVAL_CASES, eval_hats, eval_knobs, load_golden
from oracle import quant as Q
from oracle.attention import causal_attention_pure, prefill_eval as oracle_eval

pytestmark = pytest.mark.gpu
F16, F32 = np.float16, np.float32


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _strict(out, ref):
    out, ref = np.asarray(out, F32), np.asarray(ref, F32)
    ulp = np.spacing(np.maximum(np.abs(ref), np.abs(out)).astype(F16)).astype(F32)
    return np.abs(out - ref) <= np.maximum(2 * ulp, 5e-4)


def _bar(out, ref, sel, V, Vh, k_corr, grp, *, rows=None, max_frac=0.02, base=None):
    """out / ref (T, Hq, D); sel {(h, t): token indices}; V / Vh (Hkv, T, D).
    Rows (h, t) in ``rows`` (all by default) are within ``base`` (default
    max(2 ulps, 5e-4)) plus the weight-rounding allowance; at most
    ``max_frac`` of them need the allowance."""
    out, ref = np.asarray(out, F32), np.asarray(ref, F32)
    ulp = np.spacing(np.maximum(np.abs(ref), np.abs(out)).astype(F16)).astype(F32)
    if base is None:
        base = np.maximum(2 * ulp, 5e-4)
    err = np.abs(out - ref)
    rv = (V.astype(F32) - Vh.astype(F32)).astype(F16).astype(F32)
    rows = sorted(sel) if rows is None else sorted(rows)
    need = 0
    for h, t in rows:
        if np.all(err[t, h] <= base[t, h]):
            continue
        need += 1
        idx, hk = np.asarray(sel[(h, t)]), h // grp
        allow = (2.0 ** -11 * (np.abs(rv[hk, idx]) + 2 * k_corr * np.abs(Vh[hk, idx].astype(F32) - ref[t, h]))).sum(0)
        assert np.all(err[t, h] <= base[t, h] + allow), (h, t, float(err[t, h].max()))
    assert need <= max(1, int(max_frac * len(rows))), (need, len(rows))


def _device_eval(Qh, K, V, Kh, Vh, knobs, diag_cap):
    """Qh (Hq, T, D), the rest (Hkv, T, D) numpy fp16 -> (out (T, Hq, D),
    diag (Hq, T, cap), the base output (Hq, T, D))."""
    import care_kv
    d = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (Qh, K, V, Kh, Vh)]
    O = care_kv.prefill_attention(d[0], d[3], d[4])
    out, diag = care_kv.prefill_eval(*d, O, diag_cap=diag_cap, **knobs)
    torch.cuda.synchronize()
    return out.cpu().numpy().transpose(1, 0, 2), diag.cpu().numpy(), O.cpu().numpy()


def _check_against_oracle(Qh, K, V, Kh, Vh, knobs, *, max_flips=None):
    """Selections equal the oracle's up to near-ties; outputs meet the bar
    against the oracle run with the device's selections."""
    Hq, T, _ = Qh.shape
    out, dg, O = _device_eval(Qh, K, V, Kh, Vh, knobs, T)
    diag = {}
    oracle_eval(Qh, K, V, Kh, Vh, diag=diag, o_base=O, **knobs)
    force, sel = {}, {}
    for (h, t), (idx, sc) in diag.items():
        got = dg[h, t]
        got = got[got >= 0]
        assert len(got) == len(idx), (h, t, len(got), len(idx))
        assert np.all(np.diff(got) > 0) and (len(got) == 0 or got[-1] <= t), (h, t)
        sel[(h, t)] = got
        if not np.array_equal(got, idx):
            # a flip swaps tokens whose scores tie to within 1e-5 of the row's top score
            tol = 1e-5 * float(np.abs(sc).max()) + 1e-30
            assert abs(float(sc[got].min()) - float(sc[idx].min())) <= tol, (h, t)
            force[(h, t)] = got
    flips = len(force)
    print(f"  {flips} near-tie selection differences of {len(diag)} rows", flush=True)
    assert flips <= (max_flips if max_flips is not None else max(2, len(diag) // 50)), (flips, len(diag))
    ref = oracle_eval(Qh, K, V, Kh, Vh, force_sel=force, o_base=O, **knobs)
    _bar(out, ref, sel, V, Vh, knobs["k_corr_scale"], Hq // K.shape[0])
    return out, dg, sel, force, O


@pytest.mark.parametrize("name", sorted(EVAL_CASES))
def test_prefill_eval_reference_golden(name):
    """The reference's carekv_eval goldens (GQA 4 at D = 64 with both kinds
    normalised; MHA at D = 128 with the K kind alone, min_residuals 2; GQA 2
    at D = 128 with the V kind alone, min_residuals 2) against the oracle and
    against the golden output."""
    print(f"carekv_eval golden {name}", flush=True)
    g = load_golden(f"prefill_{name}.npz")
    spec = EVAL_CASES[name]
    T = int(g["T"])
    Kh, Vh = eval_hats(g, spec)
    Qh = g["Q"].transpose(1, 0, 2)
    kn = eval_knobs(g)
    out, _, sel, force, O = _check_against_oracle(Qh, g["K"][:, :T], g["V"][:, :T], Kh, Vh, kn)
    same = {r for r in sel if r not in force}
    ref = g["O"].astype(F32)
    base_diff = np.abs(O.astype(F32) - causal_attention_pure(Qh, Kh, Vh)[0].astype(F32)).transpose(1, 0, 2)
    ulp = np.spacing(np.maximum(np.abs(ref), np.abs(out.astype(F32))).astype(F16)).astype(F32)
    _bar(out, ref, sel, g["V"][:, :T], Vh, kn["k_corr_scale"], spec["Hq"] // spec["Hkv"], rows=same, max_frac=1.0,
         base=base_diff + ulp + 1e-6)
    assert np.linalg.norm(out.astype(F32) - ref) <= 1e-2 * np.linalg.norm(ref)


def _rand_case(Hq, Hkv, D, T, seed, bits=2):
    rng = np.random.default_rng(seed)
    K = (rng.standard_normal((Hkv, T, D)) * np.exp(0.6 * rng.standard_normal((Hkv, 1, D)))).astype(F16)
    V = (rng.standard_normal((Hkv, T, D)) * np.exp(0.4 * rng.standard_normal((Hkv, T, 1)))).astype(F16)
    Qh = (rng.standard_normal((Hq, T, D)) * 0.7).astype(F16)
    Kh = Q.dequantize(*Q.quantize(K, bits, 32), 32)
    Vh = Q.dequantize(*Q.quantize(V, bits, 32), 32)
    return Qh, K, V, Kh, Vh


KNOBS = {
    "both-norm": dict(ratio=0.04, min_residuals=1, kind="both", v_score="output_aware", normalize=True,
                      k_corr_scale=0.1),
    "both-raw": dict(ratio=0.1, min_residuals=3, kind="both", v_score="norm", normalize=False, k_corr_scale=0.5),
    "v": dict(ratio=0.02, min_residuals=1, kind="v", v_score="output_aware", normalize=False, k_corr_scale=0.1),
    "k": dict(ratio=0.05, min_residuals=0, kind="k", v_score="output_aware", normalize=False, k_corr_scale=0.3),
}


@pytest.mark.parametrize("knob", sorted(KNOBS))
@pytest.mark.parametrize("Hq,Hkv,D,T", [(8, 2, 128, 300), (3, 1, 64, 529)], ids=["gqa4-d128-t300", "gqa3-d64-t529"])
def test_prefill_eval_random(knob, Hq, Hkv, D, T):
    """2-bit hats, rows past one work-group's 256 threads (several scores a
    thread in the selection), every knob set."""
    print(f"carekv_eval random {knob} Hq={Hq} Hkv={Hkv} D={D} T={T}", flush=True)
    _check_against_oracle(*_rand_case(Hq, Hkv, D, T, seed=T + D + len(knob)), KNOBS[knob])


def test_prefill_eval_budget_edges():
    """ratio 0 with min_residuals 0 selects nothing (the output is the base
    output, bit for bit); ratio 1 selects every token; exact hats (zero
    residuals) tie every score at 0: the lowest indices are taken and the
    output is the base output."""
    import care_kv
    print("carekv_eval budget edges", flush=True)
    Qh, K, V, Kh, Vh = _rand_case(4, 2, 64, 140, seed=9)
    base = dict(v_score="output_aware", normalize=True, k_corr_scale=0.1, kind="both")
    d = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (Qh, K, V, Kh, Vh)]
    O = care_kv.prefill_attention(d[0], d[3], d[4])
    out, dg = care_kv.prefill_eval(*d, O, ratio=0.0, min_residuals=0, diag_cap=4, **base)
    assert torch.equal(out, O) and bool((dg == -1).all())
    _, dg, _, _, _ = _check_against_oracle(Qh, K, V, Kh, Vh, dict(base, ratio=1.0, min_residuals=1), max_flips=0)
    for t in range(140):
        assert np.array_equal(dg[:, t, :t + 1], np.broadcast_to(np.arange(t + 1), (4, t + 1)))
    out, dg = care_kv.prefill_eval(d[0], d[1], d[2], d[1], d[2], O, ratio=0.05, min_residuals=2, diag_cap=8,
                                   **base)
    assert torch.equal(out, O)
    dg = dg.cpu().numpy()
    for t in range(140):
        k = min(max(2, int((t + 1) * 0.05)), t + 1)
        assert np.array_equal(dg[:, t, :k], np.broadcast_to(np.arange(k), (4, k))), t


def test_prefill_eval_batch_and_layer(monkeypatch):
    """A batch of two sequences equals each sequence alone; the layer in
    carekv_eval mode (identity projections, so the layer output is the
    corrected attention) equals the direct call over its own hats."""
    import care_kv
    print("carekv_eval batch + layer", flush=True)
    knobs = KNOBS["both-norm"]
    cases = [_rand_case(4, 2, 64, 96, seed=s, bits=3) for s in (21, 22)]
    d = [torch.from_numpy(np.stack([c[i] for c in cases])).cuda() for i in range(5)]
    O = care_kv.prefill_attention(d[0], d[3], d[4])
    both = care_kv.prefill_eval(*d, O, **knobs)
    for b in range(2):
        one = care_kv.prefill_eval(*(x[b] for x in d), O[b], **knobs)
        assert torch.equal(both[b], one), b
    # the layer: hidden = [q; k; v] with identity projections
    monkeypatch.setenv("CAREKV_PREFILL_MODE", "carekv_eval")
    monkeypatch.setenv("CAREKV_PREFILL_RESIDUAL_RATIO", str(knobs["ratio"]))
    monkeypatch.setenv("CAREKV_PREFILL_MIN_RESIDUALS", str(knobs["min_residuals"]))
    monkeypatch.setenv("CAREKV_PREFILL_RESIDUAL_KIND", knobs["kind"])
    monkeypatch.setenv("CAREKV_V_SCORE", knobs["v_score"])
    monkeypatch.setenv("CAREKV_SCORE_NORMALIZE", "1")
    monkeypatch.setenv("CAREKV_K_CORRECTION_SCALE", str(knobs["k_corr_scale"]))
    Hq, Hkv, D, T = 4, 2, 64, 96
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16, max_pages=10,
                              base_bits=3, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                              packed_base=True, scale_quant="int8", store_budget_mode="ratio",
                              store_budget_ratio=0.03, read_budget_ratio=0.0)
    nq, nk = Hq * D, Hkv * D
    eye = torch.eye(nq + 2 * nk, dtype=torch.float16, device="cuda")
    lay = care_kv.CAREKVLayer(cfg, 0, eye[:nq].contiguous(), eye[nq:nq + nk].contiguous(),
                              eye[nq + nk:].contiguous(), eye[:nq, :nq].contiguous())
    Qh, K, V = (torch.from_numpy(x) for x in cases[0][:3])
    hidden = torch.cat([Qh.permute(1, 0, 2).reshape(T, -1), K.permute(1, 0, 2).reshape(T, -1),
                        V.permute(1, 0, 2).reshape(T, -1)], 1).cuda()
    cache = care_kv.CAREKVCache(cfg, n_seq=1)
    out = lay.prefill(cache, hidden).reshape(T, Hq, D).transpose(0, 1)
    Khat = care_kv.quant_dequant(K.cuda(), 3, 32)
    Vhat = care_kv.quant_dequant(V.cuda(), 3, 32)
    O1 = care_kv.prefill_attention(Qh.cuda(), Khat, Vhat)
    ref = care_kv.prefill_eval(Qh.cuda(), K.cuda(), V.cuda(), Khat, Vhat, O1, **knobs)
    assert torch.equal(out, ref)


def test_prefill_eval_max_length():
    """T = 8192, the longest prompt (the score arrays take 64 KiB of dynamic
    LDS): rows before 512 see only the first 512 tokens, so they equal, bit
    for bit, a T = 512 run over that prefix, which is itself checked against
    the oracle; the last rows are finite and select k = max(1, int((t + 1)
    ratio)) ascending tokens at or before the row."""
    import care_kv
    T, n = 8192, 512
    print(f"carekv_eval max length T={T}", flush=True)
    Qh, K, V, Kh, Vh = _rand_case(2, 1, 64, T, seed=23)
    knobs = dict(ratio=0.02, min_residuals=1, kind="both", v_score="output_aware", normalize=False,
                 k_corr_scale=0.1)
    d = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (Qh, K, V, Kh, Vh)]
    O = care_kv.prefill_attention(d[0], d[3], d[4])
    out, dg = care_kv.prefill_eval(*d, O, diag_cap=200, **knobs)
    dp = [x[:, :n].contiguous() for x in d]
    Op = care_kv.prefill_attention(dp[0], dp[3], dp[4])
    outp, dgp = care_kv.prefill_eval(*dp, Op, diag_cap=200, **knobs)
    torch.cuda.synchronize()
    assert torch.equal(O[:, :n], Op)
    assert torch.equal(out[:, :n], outp) and torch.equal(dg[:, :n], dgp)
    assert bool(torch.isfinite(out.float()).all())
    dg = dg.cpu().numpy()
    for t in (n, 4095, 4096, T - 2, T - 1):
        k = min(max(1, int((t + 1) * knobs["ratio"])), t + 1)
        for h in range(2):
            got = dg[h, t]
            assert np.all(got[:k] >= 0) and np.all(np.diff(got[:k]) > 0) and got[k - 1] <= t, (h, t)
            assert np.all(got[k:] == -1), (h, t)
    _check_against_oracle(Qh[:, :n], K[:, :n], V[:, :n], Kh[:, :n], Vh[:, :n], knobs)


def test_prefill_eval_max_length_d128():
    """T = 8192 at head_dim 128 (64 KiB of dynamic score arrays plus the
    kernel's static LDS): sampled long rows of both query heads against the
    oracle restricted to those rows, over the same base output (selections
    up to near-ties, outputs under the bar)."""
    import care_kv
    T, Hq, Hkv, D = 8192, 2, 1, 128
    rows = [511, 4095, 6000, T - 1]
    print(f"carekv_eval max length D={D} T={T} rows={rows}", flush=True)
    Qh, K, V, Kh, Vh = _rand_case(Hq, Hkv, D, T, seed=29)
    knobs = dict(ratio=0.01, min_residuals=1, kind="both", v_score="output_aware", normalize=True,
                 k_corr_scale=0.1)
    d = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (Qh, K, V, Kh, Vh)]
    O = care_kv.prefill_attention(d[0], d[3], d[4])
    out, dg = care_kv.prefill_eval(*d, O, diag_cap=128, **knobs)
    torch.cuda.synchronize()
    out = out.cpu().numpy().transpose(1, 0, 2)
    dg, O = dg.cpu().numpy(), O.cpu().numpy()
    assert np.isfinite(out.astype(F32)).all()
    diag = {}
    oracle_eval(Qh, K, V, Kh, Vh, diag=diag, o_base=O, rows=rows, **knobs)
    force, sel = {}, {}
    for (h, t), (idx, sc) in diag.items():
        got = dg[h, t]
        got = got[got >= 0]
        assert len(got) == len(idx) == max(1, int((t + 1) * knobs["ratio"])), (h, t, len(got), len(idx))
        sel[(h, t)] = got
        if not np.array_equal(got, idx):
            tol = 1e-5 * float(np.abs(sc).max()) + 1e-30
            assert abs(float(sc[got].min()) - float(sc[idx].min())) <= tol, (h, t)
            force[(h, t)] = got
    assert len(force) <= 2, len(force)
    ref = oracle_eval(Qh, K, V, Kh, Vh, force_sel=force, o_base=O, rows=rows, **knobs)
    _bar(out, ref, sel, V, Vh, knobs["k_corr_scale"], Hq // Hkv, rows=sorted(sel), max_frac=0.25)


def test_prefill_eval_rejects_non_finite_ratio():
    """An infinite or NaN ratio raises before any kernel runs (Python's
    int(n * ratio) raises there, layer.py:397); a huge finite ratio keeps
    every token, as int(n * ratio) >= n does."""
    import care_kv
    print("carekv_eval ratio edges", flush=True)
    Qh, K, V, Kh, Vh = _rand_case(2, 1, 64, 40, seed=31)
    d = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (Qh, K, V, Kh, Vh)]
    O = care_kv.prefill_attention(d[0], d[3], d[4])
    base = dict(min_residuals=1, kind="both", v_score="output_aware", normalize=False, k_corr_scale=0.1)
    for bad in (float("inf"), float("nan")):
        with pytest.raises(care_kv.CarekvError, match="finite"):
            care_kv.prefill_eval(*d, O, ratio=bad, **base)
    _, dg = care_kv.prefill_eval(*d, O, ratio=1e300, diag_cap=40, **base)
    _, dg1 = care_kv.prefill_eval(*d, O, ratio=1.0, diag_cap=40, **base)
    assert torch.equal(dg, dg1)
    dg = dg.cpu().numpy()
    for t in range(40):
        assert np.array_equal(dg[:, t, :t + 1], np.broadcast_to(np.arange(t + 1), (2, t + 1))), t
