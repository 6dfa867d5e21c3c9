"""The wave-per-query select against the work-group select (needs a GPU).

decode_select_wave_kernel takes rows of at most 256 pages with one K and
one V slot per page (prompt rows of the prefill correction, short decode
rows) and reduces every float sum in the work-group form's order, so both
forms must give the same outputs and selections bit for bit.  The cases
cover prefill rows (GQA 8, two rows per entry), decode rows of 1-256 pages
(GQA 8 through the 16-column streaming kernel, MHA and GQA 4 through the
4-query one), the joint and separate policies, normalised and raw scores,
ratio and absolute budgets, ties at the threshold (repeated pages), and
correction with the linear K mode.  CAREKV_SELECT_WAVE=2 takes the wave
form for every row it covers, =0 the work-group form; both are held to the
oracle elsewhere.
"""
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
    monkeypatch.setenv("CAREKV_K_CORRECTION_MODE", "exact")
    return monkeypatch


def _both(env, fn):
    env.setenv("CAREKV_SELECT_WAVE", "2")  # the wave form for every row it covers
    a = fn()
    torch.cuda.synchronize()
    env.setenv("CAREKV_SELECT_WAVE", "0")
    b = fn()
    torch.cuda.synchronize()
    return a, b


def _same(a, b):
    for x, y in zip(a, b):
        if x.dtype == torch.float16:
            x, y = x.view(torch.int16), y.view(torch.int16)
        assert torch.equal(x, y)


DECODE_CASES = [
    # Hq, Hkv, D, lengths, (read K, read V), policy, normalise, ratio budget
    (32, 4, 64, [512, 40, 300], (32, 32), "joint", "1", None),
    (8, 8, 128, [4096, 1000, 17], (64, 64), "joint", "1", None),
    (16, 4, 128, [2000, 3001], (16, 24), "separate", "1", None),
    (16, 4, 128, [2000, 777], (16, 24), "joint", "0", None),
    (8, 2, 64, [1500], (0, 0), "joint", "1", 0.05),
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=[f"g{c[0] // c[1]}-D{c[2]}-{c[5]}-n{c[6]}" for c in DECODE_CASES])
def test_wave_select_decode_matches(paper_env, case):
    import care_kv
    Hq, Hkv, D, lens, (rk, rv), pol, norm, ratio = case
    print(f"wave select decode Hq={Hq} Hkv={Hkv} D={D} lens={lens} {pol} norm={norm}", flush=True)
    paper_env.setenv("CAREKV_SCORE_NORMALIZE", norm)
    dev = torch.device("cuda", 0)
    budget = dict(read_budget_mode="absolute", read_abs_k=rk, read_abs_v=rv) if ratio is None else \
        dict(read_budget_mode="ratio", read_budget_ratio=ratio)
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                              max_pages=max(lens) // 16 + 4, base_bits=3, group_size=32, k_channel_group=32,
                              v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8",
                              store_budget_mode="ratio", store_budget_ratio=0.03, route_policy=pol,
                              **({"read_budget_ratio": 0.0} if ratio is None else {}), **budget)
    cache = care_kv.CAREKVCache(cfg, device=dev, n_seq=len(lens))
    g = torch.Generator(device=dev).manual_seed(11 + D + Hq)
    for b, n in enumerate(lens):
        K = torch.randn(Hkv, n, D, generator=g, device=dev)
        K[:, :, :2] *= 6.0
        V = torch.randn(Hkv, n, D, generator=g, device=dev)
        if b == 0 and n >= 64:  # equal pages: equal K and V scores, ties at the threshold
            K[:, 32:48] = K[:, 16:32]
            V[:, 32:48] = V[:, 16:32]
        cache.write_prefill(0, K.half(), V.half(), seqs=[b])
    q = torch.randn(len(lens), Hq, D, generator=g, device=dev).half()
    a, b = _both(paper_env, lambda: care_kv.decode_attention(cache, 0, q, diag_cap=512))
    _same(a, b)
    assert int((a[1] >= 0).sum()) > 0


@pytest.mark.parametrize("k_mode", ["exact", "linear"])
def test_wave_select_prefill_rows_match(paper_env, k_mode):
    import care_kv
    paper_env.setenv("CAREKV_K_CORRECTION_MODE", k_mode)
    dev = torch.device("cuda", 0)
    T, Hq, Hkv, D = 1100, 32, 4, 64
    cfg = care_kv.CacheConfig(num_layers=1, num_heads=Hq, num_kv_heads=Hkv, head_dim=D, page_size=16,
                              max_pages=T // 16 + 4, base_bits=3, group_size=32, k_channel_group=32,
                              v_token_block=4, sketch_dim=32, packed_base=True, scale_quant="int8",
                              store_budget_mode="ratio", store_budget_ratio=0.03, read_budget_ratio=0.0,
                              read_budget_mode="absolute", read_abs_k=16, read_abs_v=16, route_policy="joint")
    cache = care_kv.CAREKVCache(cfg, device=dev)
    g = torch.Generator(device=dev).manual_seed(5)
    K = torch.randn(Hkv, T, D, generator=g, device=dev).half()
    V = torch.randn(Hkv, T, D, generator=g, device=dev).half()
    cache.write_prefill(0, K, V)
    Kh, Vh = care_kv.quant_dequant(K, 3, 32), care_kv.quant_dequant(V, 3, 32)
    Q = torch.randn(T, Hq, D, generator=g, device=dev).half()
    _, lse = care_kv.prefill_attention(Q.transpose(0, 1), Kh, Vh, return_lse=True)
    a, b = _both(paper_env, lambda: care_kv.prefill_correction(cache, 0, Q, Kh, Vh, lse, diag_cap=64,
                                                               rows_per_call=300))
    _same(a, b)
    d = a[1].cpu().numpy()
    assert (d[:, :, 0] >= 0).mean() > 0.5
