"""The packed KIVI base (CacheConfig.kivi_packed, no reference counterpart) on
the GPU: the reference keeps the KIVI-style 2-bit base as fp16 K_hat / V_hat
side-buffer pages (cache.py:487-499); here the prompt's full pages hold
2-bit codes (K against one per-channel scale vector, V against per-token
scales) and only the later rows stay fp16.

The format is pinned by what it must reproduce: carekv_kivi_codes against
the oracle's kivi_codes (codes and scales bit for bit), the K_hat / V_hat
rows the packed cache reads back against the side-buffer cache's (and the
reference golden's), the page metadata and residual slots byte for byte
against the reference golden, and the decode output against the
reference's under the golden bars (tests/test_gpu_parity.py:check_decode).
Against the side-buffer cache on the same inputs: the same metadata and
slots byte for byte; logits equal up to fp32 summation order (K on the MFMA
as integer codes against q * scale in fp16 hi + lo), so selections equal up
to epsilon ties; outputs within 2e-3 or two fp16 ulps, since the packed
prefix runs the 4-query-head kernel, whose V product carries the V scales
on fp16 weights, while the side buffer runs the generic fp16 kernel (each
within the golden bar of the reference).
"""
import numpy as np
import pytest
import torch

from helpers import DECODE_CASES, case_cfg_kwargs, load_golden
from oracle import quant as Q

pytestmark = pytest.mark.gpu
F16, F32 = np.float16, np.float32


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


@pytest.fixture
def paper_env(monkeypatch):
    from helpers import PAPER_ENV
    for k, v in PAPER_ENV.items():
        monkeypatch.setenv(k, v)
    return monkeypatch


def _same_values(got, ref):
    """Equal as numbers (+0 == -0), NaN exactly where ref has NaN."""
    got, ref = np.asarray(got).astype(F32), np.asarray(ref).astype(F32)
    nan = np.isnan(ref)
    return np.array_equal(np.isnan(got), nan) and np.array_equal(got[~nan], ref[~nan])


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_kivi_codes_match_oracle(bits):
    import care_kv
    print(f"carekv_kivi_codes bits={bits}", flush=True)
    rng = np.random.default_rng(10 + bits)
    X = (rng.standard_normal((3, 70, 128)) * np.exp(rng.standard_normal((1, 1, 128)))).astype(F16)
    X[1, :, 5] = 0
    X[2, 9, :] = 0
    xd = torch.from_numpy(X).cuda()
    for per_channel in (True, False):
        codes, scale = care_kv.kivi_codes(xd, bits, per_channel)
        rc, rs = Q.kivi_codes(X, bits, per_channel)
        assert np.array_equal(codes.cpu().numpy(), rc), per_channel
        rs = rs[:, 0, :] if per_channel else rs[..., 0]
        s = scale.cpu().numpy()
        assert np.array_equal(np.isnan(s), np.isnan(rs)) and np.array_equal(s.view(np.uint16)[~np.isnan(rs)],
                                                                           rs.view(np.uint16)[~np.isnan(rs)])
        deq = (codes.float() * (scale.float().unsqueeze(-2) if per_channel else scale.float().unsqueeze(-1)))
        assert _same_values(deq.half().cpu().numpy(), Q.kivi_qdq(X, bits, per_channel)), per_channel


def _build(g, spec, packed, **over):
    import care_kv
    kw = dict(case_cfg_kwargs(g, spec), **over)
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0, compat=True,
                              kivi_packed=packed, **kw)
    cache = care_kv.CAREKVCache(cfg, device="cuda")
    T, n_app = int(g["T"]), int(g["n_append"])
    K = torch.from_numpy(g["K"]).cuda()
    V = torch.from_numpy(g["V"]).cuda()
    cache.write_prefill(0, K[:, :T], V[:, :T])
    for t in range(T, T + n_app):
        cache.append(0, K[:, t], V[:, t])
    torch.cuda.synchronize()
    return cache


def _meta_equal(a, b):
    """Page metadata and residual slots of two caches, byte for byte."""
    for nm in ("valid", "has_meta", "k_slot", "v_slot", "k_err", "v_err", "k_sketch", "v_sq", "next_slot",
               "k_res", "k_res_scale", "v_res", "v_res_scale"):
        x, y = getattr(a, nm).cpu(), getattr(b, nm).cpu()
        assert torch.equal(x.view(torch.uint8) if x.dtype != torch.float32 else x.view(torch.int32),
                           y.view(torch.uint8) if y.dtype != torch.float32 else y.view(torch.int32)), nm


def test_packed_kivi_golden_decode(paper_env):
    """The reference's KIVI decode golden (gqa4_d128_kivi: 2-bit K per
    channel over the prompt, V per token, decode appends past the prompt's
    partial last page) replayed into a packed cache: read-back K_hat / V_hat
    equal the golden side buffer's, metadata and slots equal the side-buffer
    cache's, the decode output meets the golden bars."""
    import care_kv
    from test_gpu_parity import build_oracle_case, check_decode
    name = "gqa4_d128_kivi"
    g = load_golden(f"decode_{name}.npz")
    spec = DECODE_CASES[name]
    print(f"packed KIVI golden {name}", flush=True)
    packed, side = _build(g, spec, True), _build(g, spec, False)
    assert packed.kivi_packed and int(packed.n_packed[0]) == int(g["T"]) // 16
    for h in range(spec["Hkv"]):
        kp, vp, lp = packed.read_base_hat_concat(0, h)
        ks, vs, ls = side.read_base_hat_concat(0, h)
        assert lp == ls
        assert _same_values(kp.cpu().numpy(), ks.cpu().numpy()), h
        assert _same_values(vp.cpu().numpy(), vs.cpu().numpy()), h
        valid = g["valid"][h]
        ref_k = np.concatenate([g["K_hat"][h, p, :n] for p, n in enumerate(valid) if n])
        assert _same_values(kp.cpu().numpy(), ref_k), h
    _meta_equal(packed, side)
    oc, _ = build_oracle_case(g, name)
    check_decode(packed, oc, spec, g["Q"], g["O"], paper_env, spec["k_mode"])


def _random_pair(Hq, Hkv, D, T, n_app, seed, tail_pages=0):
    import care_kv
    rng = np.random.default_rng(seed)
    K = (rng.standard_normal((Hkv, T + n_app, D)) * np.exp(0.7 * rng.standard_normal((Hkv, 1, D)))).astype(F16)
    V = (rng.standard_normal((Hkv, T + n_app, D)) * np.exp(0.5 * rng.standard_normal((Hkv, T + n_app, 1)))).astype(F16)
    K[0, :, 3] = 0  # an all-zero channel: NaN K_hat in the reference's base
    kw = dict(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
              max_pages=(T + n_app) // 16 + 2, base_bits=2, group_size=32, k_channel_group=32, v_token_block=4,
              sketch_dim=32, base_quantizer="kivi_style", store_budget_mode="absolute", store_abs_k=2,
              store_abs_v=4, read_budget_mode="absolute", read_abs_k=6, read_abs_v=6, route_policy="joint",
              packed_base=True, read_budget_ratio=0.0)
    caches = []
    for packed in (True, False):
        cfg = care_kv.CacheConfig(kivi_packed=packed, kivi_tail_pages=tail_pages, **kw)
        c = care_kv.CAREKVCache(cfg, device="cuda", n_seq=2)
        Kd, Vd = torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda()
        # two sequences: the prompt and its first 5 rows shorter
        c.write_prefill(0, Kd[None, :, :T], Vd[None, :, :T], seqs=[0])
        c.write_prefill(0, Kd[None, :, :T - 5], Vd[None, :, :T - 5], seqs=[1])
        for t in range(n_app):
            c.append(0, torch.stack([Kd[:, T + t], Kd[:, T - 5 + t]]), torch.stack([Vd[:, T + t], Vd[:, T - 5 + t]]))
        caches.append(c)
    torch.cuda.synchronize()
    return caches


@pytest.mark.parametrize("Hq,Hkv,D", [(8, 2, 128), (4, 4, 64)], ids=["gqa4-d128", "mha-d64"])
@pytest.mark.parametrize("live", [True, False], ids=["kscore", "proxy"])
def test_packed_kivi_matches_side_buffer(paper_env, Hq, Hkv, D, live):
    """Random 2-bit KIVI caches (two sequences, prompts of 203 and 198 rows,
    37 decode appends each, an all-zero K channel): the packed and the
    side-buffer cache hold the same metadata and slots, and decode to the
    same output and selections (exact K correction, the query-aware K score
    or the sketch proxy)."""
    import care_kv
    print(f"packed vs side-buffer KIVI Hq={Hq} Hkv={Hkv} D={D} live={live}", flush=True)
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    paper_env.setenv("CAREKV_KSCORE_LIVE", "1" if live else "0")
    packed, side = _random_pair(Hq, Hkv, D, 203, 37, seed=Hq * 7 + D + int(live))
    assert packed.n_packed.tolist() == [12, 12]
    _meta_equal(packed, side)
    rng = np.random.default_rng(5)
    q = torch.from_numpy(rng.standard_normal((2, Hq, D)).astype(F16)).cuda()
    outs = [care_kv.decode_attention(c, 0, q, diag_cap=512) for c in (packed, side)]
    base = [care_kv.decode_attention(c, 0, q, correction=False) for c in (packed, side)]
    for (o_p, d_p), (o_s, d_s) in [outs] + [((base[0], None), (base[1], None))]:
        o_p, o_s = o_p.float().cpu().numpy(), o_s.float().cpu().numpy()
        nan = np.isnan(o_s)
        assert np.array_equal(np.isnan(o_p), nan)
        ulp = np.spacing(np.abs(o_s[~nan]).astype(F16)).astype(F32)
        assert np.all(np.abs(o_p[~nan] - o_s[~nan]) <= np.maximum(2e-3, 2 * ulp))
    d_p, d_s = outs[0][1].cpu().numpy(), outs[1][1].cpu().numpy()
    rows = d_p.shape[0] * d_p.shape[1]
    differ = int(sum(not np.array_equal(a, b) for a, b in zip(d_p.reshape(rows, -1), d_s.reshape(rows, -1))))
    assert differ * 16 <= rows, differ


def test_packed_kivi_tail_capacity():
    """kivi_tail_pages bounds the fp16 rows: an append past it is refused
    before any kernel runs."""
    import care_kv
    packed, _ = _random_pair(8, 2, 128, 40, 0, seed=3, tail_pages=2)
    k = torch.zeros(2, 2, 128, dtype=torch.float16, device="cuda")
    for _ in range(24):  # page 2 (the prompt's partial page) fills, page 3 is the second tail page
        packed.append(0, k, k)
    with pytest.raises(care_kv.CarekvError, match="tail full"):
        for _ in range(16):
            packed.append(0, k, k)
