"""The analysis utilities of the package API (utils.py of the reference),
against closed forms worked by hand, and the token-importance probe against
a uniform-attention closed form (CPU)."""
import math

import numpy as np
import pytest
import torch



def test_estimate_memory_bytes_closed_form():
    import care_kv
    cfg = care_kv.CacheConfig(num_layers=2, num_heads=8, num_kv_heads=2, head_dim=128, base_bits=3, group_size=32,
                              packed_base=True, scale_quant="int8", store_budget_ratio=0.03)
    m = care_kv.estimate_memory_bytes(cfg, 1000)
    # 1000 tokens -> 63 pages of 16 = 1008 rows per (layer, kv head); 2 x 2 of them
    rows, pages = 4 * 1008, 4 * 63
    assert m["base_K_code_bytes"] == m["base_V_code_bytes"] == rows * 48      # 128 x 3 bits
    assert m["base_K_scale_bytes"] == rows * 4 + pages * 2                    # int8 per group + fp16 master
    assert m["residual_K_bytes"] == int(pages * 4 * 0.03) * (256 + 2)         # 4 K candidates a page
    assert m["residual_V_bytes"] == int(pages * 4 * 0.03) * (256 + 2)         # 4 V blocks of 4 x 128 4-bit
    assert m["metadata_bytes"] == pages * (16 + 16 + 12)
    assert m["error_norm_bytes"] == pages * 16 and m["sketch_bytes"] == pages * 4 * 32 * 2
    assert m["fp16_kv_bytes"] == 4 * 1000 * 128 * 4 and m["int4_kv_bytes"] == 4 * 1000 * 128
    parts = [k for k in m if k.endswith("_bytes") and k not in ("total_bytes", "fp16_kv_bytes", "int4_kv_bytes")]
    assert m["total_bytes"] == sum(m[k] for k in parts)
    assert m["compression_vs_fp16"] == m["total_bytes"] / m["fp16_kv_bytes"]
    f = care_kv.estimate_memory_bytes(cfg.__class__(**{**cfg.__dict__, "scale_quant": "none"}), 1000, packed=False)
    assert f["base_K_code_bytes"] == rows * 128 and f["base_K_scale_bytes"] == rows * 4 * 2 and not f["packed_mode"]


def test_sensitivity_perplexity_sweep_and_risk(capsys):
    import care_kv
    assert care_kv.calibrate_layer_sensitivity(None, [], 5) == [1.0, 0.75, 0.5, 0.75, 1.0]
    V = 37
    assert care_kv.compute_perplexity(torch.zeros(10, V), torch.arange(10) % V) == pytest.approx(V, rel=1e-6)  # fp32 loss
    calls = []
    res = care_kv.budget_sweep([0.1, 0.05], [0.02, 0.08], lambda s, r: calls.append((s, r)) or s + r)
    assert calls == [(0.1, 0.02), (0.1, 0.08), (0.05, 0.02)] and res[(0.1, 0.08)] == pytest.approx(0.18)
    assert care_kv.ABLATION_VARIANTS[0] == "base_only" and len(care_kv.ABLATION_VARIANTS) == 8
    s = torch.tensor([2.0, 1.0, 0.0])
    a = torch.tensor([0.5, 0.25, 0.25])
    st = care_kv.compute_boundary_risk_stats(s, a)
    h = -(0.5 * math.log(0.5) + 2 * 0.25 * math.log(0.25))
    assert st["min_margin"] == pytest.approx(1e-6) and st["mean_margin"] == pytest.approx((1e-6 + 1 + 2) / 3)
    assert st["max_boundary_risk"] == pytest.approx(1e6, rel=1e-6)
    assert st["attn_weighted_risk"] == pytest.approx(0.5e6 + 0.25 + 0.125, rel=1e-6)
    assert st["attention_entropy"] == pytest.approx(h) and st["effective_context_size"] == pytest.approx(math.exp(h))
    care_kv.print_memory_table(care_kv.CacheConfig(num_layers=1, num_heads=4, num_kv_heads=4), [16, 1024])
    assert "1,024" in capsys.readouterr().out


def test_importance_probe_uniform_attention():
    """q = 0 gives uniform causal attention: key n gets sum_{t >= n} 1 / (t + 1)
    from every head; Gini, normalised entropy and top-1% share of that mass."""
    import care_kv
    from care_kv import attention as A
    care_kv.reset_debug_stats()
    Hq, Hkv, T, D = 4, 2, 300, 16
    A.importance_probe(3, torch.zeros(Hq, T, D), torch.randn(Hkv, T, D))
    A.importance_probe(3, torch.zeros(Hq, T, D), torch.randn(Hkv, T, D))
    mass = Hq * np.array([sum(1.0 / (t + 1) for t in range(n, T)) for n in range(T)])
    p = mass / mass.sum()
    ent = -(p * np.log(p + 1e-12)).sum() / math.log(T)
    srt = np.sort(mass)
    gini = ((2 * np.arange(1, T + 1) - T - 1) * srt).sum() / (T * srt.sum())
    top1 = np.sort(mass)[::-1][:T // 100].sum() / mass.sum()
    got = care_kv.get_imp_per_layer()[3]
    assert got["count"] == 2
    assert got["gini"] == pytest.approx(gini, rel=1e-5) and got["norm_entropy"] == pytest.approx(ent, rel=1e-5)
    assert got["top1pct_mass"] == pytest.approx(top1, rel=1e-5)
    st = care_kv.get_debug_stats()
    assert st["imp_count"] == 2 and st["imp_gini_sum"] == pytest.approx(2 * gini, rel=1e-5)
    care_kv.reset_debug_stats()
    assert care_kv.get_imp_per_layer() == {}
