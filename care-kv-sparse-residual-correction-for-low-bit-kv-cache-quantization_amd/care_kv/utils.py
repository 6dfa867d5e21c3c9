"""Analysis utilities of the reference package's public API (utils.py):
the byte model of a cache, a layer-sensitivity heuristic, perplexity from
logits, a store/read budget sweep driver, the ablation variant list and
attention boundary-risk statistics.

These are host-side helpers: none of them runs a kernel.  The byte model
counts what the reference's layout stores (utils.py:33-151); for a
``CAREKVCache`` of this build with ``packed_base=True`` and
``scale_quant="int8"`` its base-code and base-scale bytes are the sizes of
the arena's code, scale-code and master arrays for the same pages.
"""
from __future__ import annotations

import math
from typing import Callable, Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from .config import CacheConfig


def _packed_bytes(n_values: int, bits: int) -> int:
    """Bytes of n_values tightly packed values of `bits` bits (rounded up)."""
    return -(-n_values * bits // 8)


def estimate_memory_bytes(cfg: CacheConfig, seq_len: int, store_ratio: Optional[float] = None,
                          packed: Optional[bool] = None) -> Dict[str, int]:
    """Cache bytes for one sequence of `seq_len` tokens over all layers and
    kv heads (utils.py:33-151), by component: base codes and scales, stored
    residual slots (4-bit payloads plus an fp16 scale each, `store_ratio` of
    the candidates, default cfg.store_budget_ratio), per-page metadata
    (int32 slot tables, valid count, token start and page id), fp16 error
    norms and sketches; with fp16 and INT4 K+V references and the
    compression ratios.  `packed` (default cfg.packed_base): codes packed
    at base_bits; False: one int8 per code."""
    ratio = cfg.store_budget_ratio if store_ratio is None else store_ratio
    packed = cfg.packed_base if packed is None else packed
    L, H, D = cfg.num_layers, cfg.num_kv_heads, cfg.head_dim
    n_pages = -(-seq_len // cfg.page_size)
    rows = L * H * n_pages * cfg.page_size             # token rows of whole pages
    groups = D // cfg.group_size
    code_row = _packed_bytes(D, cfg.base_bits) if packed else D
    if cfg.scale_quant == "int8":                      # int8 code per group + fp16 master per page
        scale = rows * groups + L * H * n_pages * 2
    else:
        scale = rows * groups * {"fp16": 2, "bf16": 2, "fp32": 4}.get(cfg.scale_dtype, 2)
    n_kc = D // cfg.k_channel_group
    n_vb = -(-cfg.page_size // cfg.v_token_block)
    pages = L * H * n_pages
    k_slot = _packed_bytes(cfg.page_size * cfg.k_channel_group, 4) + 2
    v_slot = _packed_bytes(cfg.v_token_block * D, 4) + 2
    res_k = int(pages * n_kc * ratio) * k_slot
    res_v = int(pages * n_vb * ratio) * v_slot
    meta = pages * (4 * n_kc + 4 * n_vb + 12)
    err = pages * 2 * (n_kc + n_vb)
    sketch = pages * n_kc * cfg.sketch_dim * 2
    base_k = base_v = rows * code_row
    total = base_k + base_v + 2 * scale + res_k + res_v + meta + err + sketch
    fp16 = L * H * seq_len * D * 4                     # K and V at 2 bytes
    int4 = L * H * seq_len * D                         # K and V at 4 bits
    return {
        "base_K_code_bytes": base_k, "base_V_code_bytes": base_v,
        "base_K_scale_bytes": scale, "base_V_scale_bytes": scale,
        "residual_K_bytes": res_k, "residual_V_bytes": res_v,
        "metadata_bytes": meta, "error_norm_bytes": err, "sketch_bytes": sketch,
        "total_bytes": total, "fp16_kv_bytes": fp16, "int4_kv_bytes": int4,
        "compression_vs_fp16": total / max(fp16, 1), "compression_vs_int4": total / max(int4, 1),
        "packed_mode": packed,
    }


def print_memory_table(cfg: CacheConfig, seq_lengths: List[int], packed: bool = True):
    """Print estimate_memory_bytes in MB for each sequence length
    (utils.py:154-175)."""
    rule = "=" * 88
    print(f"\n{rule}")
    print(f"CARE-KV Memory Estimate  (base={cfg.base_bits}bit, store_budget={cfg.store_budget_ratio:.0%}, "
          f"mode={'packed' if packed else 'int8-storage'})")
    print(rule)
    print(f"{'seq_len':>8}  {'base_MB':>8}  {'scale_MB':>9}  {'resid_MB':>9}  {'meta_MB':>8}  {'sketch_MB':>10}  "
          f"{'total_MB':>9}  {'vs_fp16':>8}")
    print("-" * 88)
    for T in seq_lengths:
        m = estimate_memory_bytes(cfg, T, packed=packed)
        mb = lambda *ks: sum(m[k] for k in ks) / 1e6  # noqa: E731
        print(f"{T:>8,}  {mb('base_K_code_bytes', 'base_V_code_bytes'):>8.2f}  "
              f"{mb('base_K_scale_bytes', 'base_V_scale_bytes'):>9.2f}  "
              f"{mb('residual_K_bytes', 'residual_V_bytes'):>9.2f}  {mb('metadata_bytes', 'error_norm_bytes'):>8.2f}  "
              f"{mb('sketch_bytes'):>10.2f}  {mb('total_bytes'):>9.2f}  {m['compression_vs_fp16']:>7.3f}x")
    print(f"{rule}\n")


def calibrate_layer_sensitivity(model_forward: Callable, calibration_inputs: List[torch.Tensor], num_layers: int,
                                device=None, hooks_enabled: bool = True) -> List[float]:
    """Per-layer sensitivity weights in (0, 1] (utils.py:182-212): the
    reference's U-shaped heuristic 0.5 + 0.5 |2 i / (L - 1) - 1| normalised
    by its maximum (the first and last layers weigh most).  The forward
    function and inputs are accepted for the reference's signature and not
    run, as there."""
    s = [0.5 + 0.5 * abs(2 * i / max(num_layers - 1, 1) - 1) for i in range(num_layers)]
    top = max(s) if s else 1.0
    return [x / top for x in s]


def compute_perplexity(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int = -100) -> float:
    """exp of the mean next-token cross entropy (utils.py:219-231): logits
    (seq_len, vocab) at position t predict targets[t + 1]."""
    loss = F.cross_entropy(logits[:-1], targets[1:], ignore_index=ignore_index, reduction="mean")
    return math.exp(loss.item())


def budget_sweep(store_ratios: List[float], read_ratios: List[float],
                 eval_fn: Callable[[float, float], float]) -> Dict[Tuple[float, float], float]:
    """eval_fn(store, read) over the grid, skipping read > store
    (utils.py:238-259); prints each point."""
    out = {}
    for sr in store_ratios:
        for rr in read_ratios:
            if rr > sr:
                continue
            out[(sr, rr)] = metric = eval_fn(sr, rr)
            print(f"  store={sr:.2%}  read={rr:.2%}  metric={metric:.4f}")
    return out


# the reference's ablation variant names (utils.py:266-275), in its order
ABLATION_VARIANTS = [
    "base_only",
    "residual_raw_error",
    "residual_attn_mass",
    "residual_k_qdotr",
    "residual_kv_separated",
    "care_kv_full",
    "care_kv_no_budget_sep",
    "care_kv_no_sketch",
]


def run_ablation(variant: str, cfg: CacheConfig, eval_fn: Callable[[CacheConfig, str], Dict]) -> Dict:
    """eval_fn(cfg, variant) for a variant of ABLATION_VARIANTS
    (utils.py:278-293)."""
    if variant not in ABLATION_VARIANTS:
        raise ValueError(f"Unknown variant: {variant}")
    print(f"\n[Ablation] Running: {variant}")
    res = eval_fn(cfg, variant)
    print(f"  Results: {res}")
    return res


def compute_attention_entropy(a: torch.Tensor) -> float:
    """Entropy in nats of attention weights a (utils.py:299-306), with the
    weights floored at 1e-10 inside the logarithm term."""
    p = a.clamp(min=1e-10)
    return float(-(p * p.log()).sum().item())


def compute_boundary_risk_stats(s: torch.Tensor, a: torch.Tensor, eps: float = 1e-6) -> Dict[str, float]:
    """Margins of the logits s to their maximum (floored at eps), the
    boundary risk 1 / margin and its attention-weighted sum, the entropy
    of a and exp(entropy) as the effective context size (utils.py:309-333)."""
    margin = (s.max() - s).clamp(min=eps)
    risk = 1.0 / margin
    h = compute_attention_entropy(a)
    return {
        "mean_margin": float(margin.mean().item()),
        "min_margin": float(margin.min().item()),
        "max_boundary_risk": float(risk.max().item()),
        "attn_weighted_risk": float((a * risk).sum().item()),
        "attention_entropy": h,
        "effective_context_size": math.exp(h),
    }
