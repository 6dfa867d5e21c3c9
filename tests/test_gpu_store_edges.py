"""Page store at the edges of its arithmetic (needs a GPU).

The store pass computes half(x / s) from one Newton step on rcp(s), and
rint through the fp16 sum q + 1536.  These tests feed it groups whose
quotients sit on both sides of every fp16 rounding boundary next to a half
integer (where a quotient off by one fp32 ulp would change the code), with
normal and subnormal group scales, and pages of tiny values whose residuals
are fp16 subnormals.  Bars: codes, scales, masters, slot ids and payload
bytes bit-exact against the oracle; error norms within one fp16 ulp;
sketches within one fp16 ulp or, where the 32-term projection cancels
(groups spanning 1e-4 .. 1e4 here), within 2^-17 of the sum of its terms'
magnitudes: twice the worst-case float32 error of a 32-term sum after a
mean, as the oracle and the kernel sum in different orders.
"""
import numpy as np
import pytest
import torch

from helpers import oracle_cache_arrays
from oracle import quant as Q
from oracle.cache import OCache, OCfg
from oracle.store import sketch_proj, write_pages_for_kv_head

pytestmark = pytest.mark.gpu

F16 = np.float16


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _ulp_diff(a, b):
    a = np.ascontiguousarray(a).astype(F16).view(np.int16).astype(np.int32)
    b = np.ascontiguousarray(b).astype(F16).view(np.int16).astype(np.int32)
    return int(np.abs(a - b).max()) if a.size else 0


def boundary_rows(rng, n_rows, D, bits):
    """fp16 rows of 32-value groups: the first value sets the group max m
    (hence the scale s = half(m / qmax)), the others are the fp16 values
    nearest to B * s and their neighbours, for B the fp16 rounding
    boundaries either side of k + 0.5 (k in the code range), |x| <= m."""
    qmax = 2 ** (bits - 1) - 1
    x = np.zeros((n_rows, D), F16)
    for r in range(n_rows):
        for g0 in range(0, D, 32):
            if rng.random() < 0.2:  # subnormal group scales
                m = F16(rng.integers(qmax, 40 * qmax) * 2.0 ** -24)
            else:
                m = F16(10.0 ** rng.uniform(-4, 4))
            s = F16(np.float32(m) / np.float32(qmax))
            grp = [m]
            while len(grp) < 32:
                k = int(rng.integers(-qmax - 1, qmax + 1))
                h = F16(k + 0.5)
                u = np.float32(np.spacing(np.abs(h)))
                b = np.float32(h) + np.float32(rng.choice([-0.5, 0.5])) * u  # fp16 midpoint next to k + 0.5
                xv = F16(b * np.float32(s))
                step = int(rng.integers(-2, 3))
                xv = (np.array([xv], F16).view(np.int16) + step).view(F16)[0]
                if np.isfinite(xv) and abs(float(xv)) <= float(m):
                    grp.append(xv)
            g = np.array(grp, F16)
            rng.shuffle(g)
            x[r, g0:g0 + 32] = g
    return x


def sketch_allowance(Kh, bits, sd, n_pages):
    """Per (page, group, k): 2^-17 * sum_c |mean_c P[c, k]| of the K
    residual column means (rows zero padded to whole pages)."""
    T, D = Kh.shape
    rows = np.zeros((n_pages * 16, D), F16)
    rows[:T] = Kh
    codes, scale = Q.quantize(rows, bits, 32)
    R = (rows.astype(np.float32) - Q.dequantize(codes, scale, 32).astype(np.float32)).astype(F16).astype(np.float64)
    Pm = np.abs(np.asarray(sketch_proj(32, sd), np.float64))
    out = np.zeros((n_pages, D // 32, sd))
    for p in range(n_pages):
        nv = min(16, T - 16 * p)
        mean = np.abs(R[16 * p:16 * p + nv].mean(0)) if nv > 0 else np.zeros(D)
        for g in range(D // 32):
            out[p, g] = mean[32 * g:32 * g + 32] @ Pm
    return out * 2.0 ** -17


def _check_slices(cache, common, K, V, H, P):
    for h in range(H):
        oc = OCache(OCfg(**{**common, "num_heads": 1, "num_kv_heads": 1}), max_slots=4 * P)
        write_pages_for_kv_head(oc, 0, 0, K[h], V[h])
        ref = oracle_cache_arrays(oc)
        for nm, t in (("K_codes", cache.kcodes), ("V_codes", cache.vcodes), ("K_scale", cache.kscale),
                      ("V_scale", cache.vscale), ("K_master", cache.kmaster), ("V_master", cache.vmaster)):
            assert np.array_equal(t[0, h, 0].cpu().numpy(), ref[nm][0]), (nm, h)
        ks, vs = cache.k_slot[0, h, 0].cpu().numpy(), cache.v_slot[0, h, 0].cpu().numpy()
        kr, vr = ref["k_slots"][0], ref["v_slots"][0]
        k0 = int(ks[ks >= 0].min()) if (ks >= 0).any() else 0
        v0 = int(vs[vs >= 0].min()) if (vs >= 0).any() else 0
        assert np.array_equal(np.where(ks >= 0, ks - k0, -1), kr), h
        assert np.array_equal(np.where(vs >= 0, vs - v0, -1), vr), h
        nk, nv = int((kr >= 0).sum()), int((vr >= 0).sum())
        assert np.array_equal(cache.k_res[0, k0:k0 + nk].cpu().numpy(), ref["k_res"][:nk]), h
        assert np.array_equal(cache.v_res[0, v0:v0 + nv].cpu().numpy(), ref["v_res"][:nv]), h
        assert np.array_equal(cache.k_res_scale[0, k0:k0 + nk].cpu().numpy(), ref["k_res_scale"][:nk, 0]), h
        assert np.array_equal(cache.v_res_scale[0, v0:v0 + nv].cpu().numpy(), ref["v_res_scale"][:nv, 0]), h
        for nm, t in (("k_err", cache.k_err), ("v_err", cache.v_err)):
            assert _ulp_diff(t[0, h, 0].cpu().numpy(), ref[nm][0]) <= 1, (nm, h)
        got = cache.k_sketch[0, h, 0].cpu().numpy().astype(np.float64)
        want = ref["k_sketch"][0].astype(np.float64)
        ulp = np.spacing(np.abs(ref["k_sketch"][0])).astype(np.float64)
        allow = np.maximum(ulp, sketch_allowance(K[h], common["base_bits"], common["sketch_dim"], P))
        bad = np.abs(got - want) > allow
        assert not bad.any(), ("k_sketch", h, np.argwhere(bad)[:4], got[bad][:4], want[bad][:4], allow[bad][:4])


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_store_quotient_boundaries(bits, D):
    import care_kv
    H, T = 2, 64
    P = T // 16
    print(f"store boundaries bits={bits} D={D}", flush=True)
    rng = np.random.default_rng(100 * bits + D)
    K = np.stack([boundary_rows(rng, T, D, bits) for _ in range(H)])
    V = np.stack([boundary_rows(rng, T, D, bits) for _ in range(H)])
    common = dict(num_layers=1, num_heads=H, num_kv_heads=H, head_dim=D, page_size=16, max_pages=P,
                  base_bits=bits, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                  store_budget_mode="absolute", store_abs_k=2, store_abs_v=2)
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0, compat=True, **common)
    cache = care_kv.CAREKVCache(cfg, device="cuda", n_seq=1)
    cache.write_prefill(0, torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda())
    torch.cuda.synchronize()
    _check_slices(cache, common, K, V, H, P)


@pytest.mark.parametrize("bits", [3, 4])
def test_store_tiny_values(bits):
    """Values a few fp16 subnormal steps wide: subnormal scales, fp16
    subnormal residuals in the error norms, sketches and payloads, a zero
    group (scale 0) and a partial last page."""
    import care_kv
    H, T, D = 2, 57, 128
    P = (T + 15) // 16
    rng = np.random.default_rng(7 + bits)
    K = (rng.integers(-60, 61, size=(H, T, D)) * 2.0 ** -24).astype(F16)
    V = (rng.integers(-9, 10, size=(H, T, D)) * 2.0 ** -24).astype(F16)
    K[0, 3, 32:64] = 0
    V[1, 5, :32] = 0
    common = dict(num_layers=1, num_heads=H, num_kv_heads=H, head_dim=D, page_size=16, max_pages=P,
                  base_bits=bits, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                  store_budget_mode="absolute", store_abs_k=2, store_abs_v=2)
    cfg = care_kv.CacheConfig(packed_base=True, scale_quant="int8", read_budget_ratio=0.0, compat=True, **common)
    cache = care_kv.CAREKVCache(cfg, device="cuda", n_seq=1)
    cache.write_prefill(0, torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda())
    torch.cuda.synchronize()
    _check_slices(cache, common, K, V, H, P)


def test_prefill_grid_ragged_starts_match_single():
    """carekv_store_prefill's device-generated jobs: a second prompt chunk
    for three sequences whose first chunks had different lengths (so each
    (sequence, kv head) starts at its own page), in one call, leaves the
    arena byte-identical to the same chunk written one sequence at a time."""
    import care_kv
    H, D = 2, 128
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=4, num_kv_heads=H, head_dim=D, page_size=16, max_pages=24,
                              base_bits=3, group_size=32, k_channel_group=32, v_token_block=4, sketch_dim=32,
                              packed_base=True, scale_quant="int8", store_budget_mode="absolute", store_abs_k=2,
                              store_abs_v=1, read_budget_ratio=0.0, compat=True)
    g = torch.Generator().manual_seed(5)
    first = [48, 16, 80]
    chunk = [torch.randn(3, H, 37, D, generator=g).half() for _ in range(2)]
    pre = [[torch.randn(H, n, D, generator=g).half() for _ in range(2)] for n in first]
    caches = []
    for batched in (True, False):
        c = care_kv.CAREKVCache(cfg, device="cuda", n_seq=3)
        for s, (k, v) in enumerate(pre):
            c.write_prefill(0, k.cuda(), v.cuda(), seqs=[s])
        if batched:
            c.write_prefill(0, chunk[0].cuda(), chunk[1].cuda(), token_start_abs=0, seqs=[0, 1, 2])
        else:
            for s in range(3):
                c.write_prefill(0, chunk[0][s:s + 1].cuda(), chunk[1][s:s + 1].cuda(), token_start_abs=0, seqs=[s])
        torch.cuda.synchronize()
        caches.append(c)
    a, b = caches
    for nm in ("kcodes", "vcodes", "kscale", "vscale", "kmaster", "vmaster", "valid", "has_meta", "k_slot", "v_slot",
               "k_err", "v_err", "k_sketch", "v_sq", "k_res", "v_res", "k_res_scale", "v_res_scale", "next_slot"):
        assert torch.equal(getattr(a, nm), getattr(b, nm)), nm
    assert np.array_equal(a.valid_host, b.valid_host) and np.array_equal(a._token_start, b._token_start)
    assert np.array_equal(a.next_page, b.next_page)
