"""Cache configuration and the CAREKV_* environment knobs.

Mirrors the reference's configuration surface so existing call sites work
unchanged: ``CacheConfig`` fields and validation (cache.py:209-384),
``apply_carekv_env_overrides`` (cache.py:51-125) and
``layer_budget_multiplier`` (cache.py:166-202).  The knobs the reference reads
inside hot functions at call time (attention.py:89-93,678,839-840;
layer.py:1148-1151; residual_store.py:104-114) are resolved here once per
call into the plain structs the kernels take.
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass
from typing import List, Optional


def apply_carekv_env_overrides(kwargs: dict) -> dict:
    """Fold CAREKV_* environment variables into CacheConfig kwargs (in place)."""
    env = os.environ

    def _set(name, key, conv):
        v = env.get(name, "")
        if v != "":
            kwargs[key] = conv(v)

    as_bool = lambda v: v == "1"  # noqa: E731
    for name, key, conv in (
        ("CAREKV_PAGE_SIZE", "page_size", int), ("CAREKV_V_TOKEN_BLOCK", "v_token_block", int),
        ("CAREKV_K_CHANNEL_GROUP", "k_channel_group", int), ("CAREKV_SKETCH_DIM", "sketch_dim", int),
        ("CAREKV_GROUP_SIZE", "group_size", int), ("CAREKV_MAX_PAGES", "max_pages", int),
        ("CAREKV_BASE_BITS", "base_bits", int), ("CAREKV_RESIDUAL_BITS", "residual_bits", int),
        ("CAREKV_STORE_BUDGET", "store_budget_ratio", float), ("CAREKV_READ_BUDGET", "read_budget_ratio", float),
        ("CAREKV_PACKED_BASE", "packed_base", as_bool), ("CAREKV_SCALE_DTYPE", "scale_dtype", str),
        ("CAREKV_SCALE_QUANT", "scale_quant", str), ("CAREKV_ROUTE_POLICY", "route_policy", str),
        ("CAREKV_STORE_BUDGET_MODE", "store_budget_mode", str), ("CAREKV_READ_BUDGET_MODE", "read_budget_mode", str),
        ("CAREKV_STORE_BUDGET_K", "store_budget_ratio_k", float), ("CAREKV_STORE_BUDGET_V", "store_budget_ratio_v", float),
        ("CAREKV_READ_BUDGET_K", "read_budget_ratio_k", float), ("CAREKV_READ_BUDGET_V", "read_budget_ratio_v", float),
        ("CAREKV_STORE_ABS_K", "store_abs_k", int), ("CAREKV_STORE_ABS_V", "store_abs_v", int),
        ("CAREKV_READ_ABS_K", "read_abs_k", int), ("CAREKV_READ_ABS_V", "read_abs_v", int),
        ("CAREKV_CORRECTION_IMPL", "correction_impl", str), ("CAREKV_PACK_IMPL", "pack_impl", str),
        ("CAREKV_BUDGET_POLICY", "budget_policy", str), ("CAREKV_VDOM_OPTIMIZED", "vdom_optimized", as_bool),
        ("CAREKV_READ_RELATIVE_THRESHOLD", "read_relative_threshold", float),
        ("CAREKV_READ_ABSOLUTE_THRESHOLD", "read_absolute_threshold", float),
        ("CAREKV_READ_MIN_KEEP", "read_min_keep", int), ("CAREKV_READ_SCORE_TEMPERATURE", "read_score_temperature", float),
        ("CAREKV_CORRECTION_NORM_CLIP", "correction_norm_clip", float),
        ("CAREKV_BASE_QUANTIZER", "base_quantizer", str), ("CAREKV_K_BITS", "k_bits_override", int),
        ("CAREKV_V_BITS", "v_bits_override", int), ("CAREKV_K_STORE_MODE", "k_store_mode", str),
        ("CAREKV_BASELINE_SCORE", "baseline_score", str),
    ):
        _set(name, key, conv)
    # no reference counterpart: CAREKV_COMPAT=1 reproduces the reference's
    # decode-path defects (CacheConfig.compat)
    _set("CAREKV_COMPAT", "compat", as_bool)
    # no reference counterpart: the packed KIVI base (CacheConfig.kivi_packed)
    _set("CAREKV_KIVI_PACKED", "kivi_packed", as_bool)
    _set("CAREKV_KIVI_TAIL_PAGES", "kivi_tail_pages", int)
    ls = env.get("CAREKV_LAYER_SENSITIVITY", "")
    if ls:
        try:
            kwargs["layer_sensitivity"] = [float(x) for x in ls.split(",") if x.strip()]
        except ValueError:
            pass
    return kwargs


@dataclass
class CacheConfig:
    """Same fields, defaults and validation as the reference CacheConfig."""
    num_layers: int = 32
    num_heads: int = 32
    num_kv_heads: Optional[int] = None
    head_dim: int = 128
    page_size: int = 16
    max_pages: int = 512
    base_bits: int = 2
    residual_bits: int = 4
    group_size: int = 64
    k_channel_group: int = 32
    v_token_block: int = 4
    store_budget_ratio: float = 0.10
    read_budget_ratio: float = 0.03
    sketch_dim: int = 32
    layer_sensitivity: Optional[List[float]] = None
    packed_base: bool = False
    packed_storage: bool = False
    scale_dtype: str = "fp16"
    scale_quant: str = "none"
    store_budget_mode: str = "ratio"
    read_budget_mode: str = "ratio"
    store_budget_ratio_k: Optional[float] = None
    store_budget_ratio_v: Optional[float] = None
    read_budget_ratio_k: Optional[float] = None
    read_budget_ratio_v: Optional[float] = None
    store_abs_k: int = 0
    store_abs_v: int = 0
    read_abs_k: int = 0
    read_abs_v: int = 0
    route_policy: str = "separate"
    vdom_optimized: bool = False
    read_relative_threshold: float = 0.0
    read_absolute_threshold: float = 0.0
    read_min_keep: int = 0
    read_score_temperature: float = 1.0
    correction_norm_clip: float = 0.0
    base_quantizer: str = "uniform"
    k_bits_override: int = -1
    v_bits_override: int = -1
    k_store_mode: str = "post_rope"
    baseline_score: str = "carekv"
    correction_impl: str = "cached"
    pack_impl: str = "vectorized"
    budget_policy: str = "uniform"
    # No reference counterpart.  compat=True reproduces three defects of the
    # reference's decode path exactly (the parity mode the reference goldens
    # run under): (i) decode_step corrects only when read_budget_ratio > 0
    # (attention.py:1025), (ii) a page the decode opens keeps a zero int8
    # scale master, so its rows read back as zero (cache.py:689-695), (iii) a
    # page the decode fills is stored with K_orig = K_hat, i.e. without slots
    # (layer.py:1088-1146); decode_step and CAREKVMultiHeadAttention then
    # select through the router's sketch-proxy score as the reference's
    # decode path does (apply_slot_corrections -> ResidualRouter.route).
    # compat=False (the default) fixes them: decode_step corrects whenever a
    # read budget is set (with the query-aware score under
    # CAREKV_KSCORE_LIVE=1), open pages are re-encoded as write_base encodes
    # their valid rows, and filled pages are stored from their true rows.
    compat: bool = False
    # No reference counterpart.  kivi_packed=True stores the kivi_style /
    # kvquant_style 2-bit base packed instead of as the reference's fp16
    # side-buffer pages (cache.py:487-499): the prompt's full pages as 2-bit
    # codes, K against one per-channel scale vector per (layer, kv head,
    # sequence), V against per-token scales, and only the later rows (the
    # prompt's partial last page, the decode rows, which the reference keeps
    # near-lossless) as fp16 K_hat / V_hat, in kivi_tail_pages pages per
    # (layer, kv head, sequence) (0: max_pages).  K_hat / V_hat, and with
    # them every output, are the side-buffer base's.
    kivi_packed: bool = False
    kivi_tail_pages: int = 0

    def __post_init__(self):
        if self.layer_sensitivity is None:
            self.layer_sensitivity = [1.0] * self.num_layers
        if self.num_kv_heads is None:
            self.num_kv_heads = self.num_heads
        if self.packed_storage and not self.packed_base:
            self.packed_base = True
        checks = (
            ("scale_dtype", {"fp16", "bf16", "fp32"}), ("scale_quant", {"none", "int8"}),
            ("store_budget_mode", {"ratio", "absolute"}),
            ("read_budget_mode", {"ratio", "absolute", "adaptive_score"}),
            ("route_policy", {"joint", "separate", "k_first", "adaptive"}),
            ("correction_impl", {"python", "cached", "vectorized"}), ("pack_impl", {"python", "vectorized"}),
            ("budget_policy", {"uniform", "u_shaped", "sensitivity", "layer_head_impact"}),
        )
        for name, allowed in checks:
            if getattr(self, name) not in allowed:
                raise ValueError(f"{name}={getattr(self, name)!r} not in {sorted(allowed)}")

    def scale_torch_dtype(self):
        import torch
        return {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[self.scale_dtype]


def layer_budget_multiplier(cfg: CacheConfig, layer_id: int) -> float:
    """Per-layer budget factor, mean 1 across layers."""
    L = cfg.num_layers
    policy = getattr(cfg, "budget_policy", "uniform")
    if policy == "uniform" or L <= 1:
        return 1.0
    if policy == "u_shaped":
        raw = [0.5 + 1.5 * abs(2 * (l / (L - 1)) - 1) for l in range(L)]
        mean = sum(raw) / L
        return raw[layer_id] / mean
    if policy == "sensitivity":
        s = cfg.layer_sensitivity or [1.0] * L
        mean = sum(s) / max(L, 1)
        return 1.0 if mean <= 0 else s[layer_id] / mean
    return 1.0  # layer_head_impact: uniform-equivalent in the reference too


# ------------------------------------------------------------------ resolution
@dataclass
class StoreKnobs:
    k_budget: int
    v_budget: int
    joint_budget: int
    joint: bool
    store_none: bool
    sensitivity: float


def resolve_store_knobs(cfg: CacheConfig, layer_id: int) -> StoreKnobs:
    """Per-page store budgets (residual_store.py:104-114, 379-419)."""
    policy = os.environ.get("CAREKV_STORE_POLICY", "residual_kind_aware").lower()
    kind = os.environ.get("CAREKV_PREFILL_RESIDUAL_KIND", "both").lower()
    mpk = int(os.environ.get("CAREKV_STORE_MIN_PER_KIND", "1"))
    kf = float(os.environ.get("CAREKV_STORE_K_FRACTION", "1.0"))
    vf = float(os.environ.get("CAREKV_STORE_V_FRACTION", "1.0"))
    if policy not in {"joint", "per_kind", "residual_kind_aware"}:
        raise ValueError(f"Unknown CAREKV_STORE_POLICY={policy}")
    if kind not in {"v", "k", "both"}:
        raise ValueError(f"Unknown CAREKV_PREFILL_RESIDUAL_KIND={kind}")
    use_k = use_v = True
    if policy == "residual_kind_aware":
        use_k, use_v = kind != "v", kind != "k"
    lm = layer_budget_multiplier(cfg, layer_id)
    n_cg = cfg.head_dim // cfg.k_channel_group
    n_vb = math.ceil(cfg.page_size / cfg.v_token_block)
    if cfg.store_budget_mode == "absolute":
        kb = int(round(max(0, int(cfg.store_abs_k)) * lm)) if use_k else 0
        vb = int(round(max(0, int(cfg.store_abs_v)) * lm)) if use_v else 0
        jb = kb + vb
    else:
        res = lambda o, fb: fb if (o is None or o < 0) else o  # noqa: E731
        rk = res(cfg.store_budget_ratio_k, cfg.store_budget_ratio) * kf * lm
        rv = res(cfg.store_budget_ratio_v, cfg.store_budget_ratio) * vf * lm
        kt, vt = max(1, n_cg), max(1, n_vb)
        kb = max(mpk, int(kt * rk)) if (use_k and rk > 0) else 0
        vb = max(mpk, int(vt * rv)) if (use_v and rv > 0) else 0
        jb = max(1, int((kt + vt) * cfg.store_budget_ratio * lm))
    none = (cfg.store_budget_ratio <= 0 and cfg.store_budget_mode != "absolute"
            and (cfg.store_budget_ratio_k or 0) <= 0 and (cfg.store_budget_ratio_v or 0) <= 0)
    return StoreKnobs(kb, vb, jb, policy == "joint", none, float(cfg.layer_sensitivity[layer_id]))


def store_caps(cfg: CacheConfig) -> tuple[int, int]:
    """Upper bound of stored K / V slots per page (record capacity)."""
    n_cg = cfg.head_dim // cfg.k_channel_group
    n_vb = math.ceil(cfg.page_size / cfg.v_token_block)
    caps_k, caps_v = 0, 0
    for l in range(cfg.num_layers):
        s = resolve_store_knobs(cfg, l)
        if s.store_none:
            continue
        if s.joint:
            caps_k = max(caps_k, min(n_cg, s.joint_budget))
            caps_v = max(caps_v, min(n_vb, s.joint_budget))
        else:
            caps_k = max(caps_k, min(n_cg, s.k_budget))
            caps_v = max(caps_v, min(n_vb, s.v_budget))
    return caps_k, caps_v


@dataclass
class ReadKnobs:
    kind: str
    joint: bool
    normalize: bool
    k_exact: bool
    k_corr_scale: float
    lambda_k: float
    lambda_v: float
    budget_ratio: bool
    abs_k: int
    abs_v: int
    ratio_k: float
    ratio_v: float
    kscore_live: bool
    route_policy: int = 0        # 0 joint/separate by `joint`, 2 k_first, 3 adaptive (route only)
    adaptive_score: bool = False  # read_budget_mode adaptive_score thresholds (route only)
    rel_threshold: float = 0.0
    abs_threshold: float = 0.0
    min_keep: int = 0


def resolve_read_knobs(cfg: CacheConfig, layer_id: int) -> ReadKnobs:
    """Read-time knobs of vectorized_joint_correction (attention.py:576-957)
    and _resolve_read_budgets (residual_router.py:37-76)."""
    kind = os.environ.get("CAREKV_PREFILL_RESIDUAL_KIND", "both").lower()
    if kind not in {"v", "k", "both"}:
        raise ValueError(f"Unknown CAREKV_PREFILL_RESIDUAL_KIND={kind}")
    mode = os.environ.get("CAREKV_K_CORRECTION_MODE", "linear").lower()
    if mode not in {"linear", "exact"}:
        raise ValueError(f"Unknown CAREKV_K_CORRECTION_MODE={mode}")
    lm = layer_budget_multiplier(cfg, layer_id)
    budget_ratio = cfg.read_budget_mode not in ("absolute", "adaptive_score")
    res = lambda o, fb: fb if (o is None or o < 0) else o  # noqa: E731
    return ReadKnobs(
        kind=kind, joint=cfg.route_policy == "joint",
        normalize=os.environ.get("CAREKV_SCORE_NORMALIZE", "0") == "1",
        k_exact=mode == "exact",
        k_corr_scale=float(os.environ.get("CAREKV_K_CORRECTION_SCALE", "0.1")),
        lambda_k=float(os.environ.get("CAREKV_KSCORE_LAMBDA_K", "1") or 1),
        lambda_v=float(os.environ.get("CAREKV_KSCORE_LAMBDA_V", "1") or 1),
        budget_ratio=budget_ratio,
        abs_k=int(round(max(0, int(cfg.read_abs_k)) * lm)),
        abs_v=int(round(max(0, int(cfg.read_abs_v)) * lm)),
        ratio_k=res(cfg.read_budget_ratio_k, cfg.read_budget_ratio) * lm,
        ratio_v=res(cfg.read_budget_ratio_v, cfg.read_budget_ratio) * lm,
        kscore_live=os.environ.get("CAREKV_KSCORE_LIVE", "0") == "1",
        route_policy={"k_first": 2, "adaptive": 3}.get(cfg.route_policy, 0),
        adaptive_score=cfg.read_budget_mode == "adaptive_score",
        rel_threshold=float(cfg.read_relative_threshold or 0.0),
        abs_threshold=float(cfg.read_absolute_threshold or 0.0),
        min_keep=int(cfg.read_min_keep or 0),
    )


def any_read_budget(cfg: CacheConfig) -> bool:
    """layer.py:813-819."""
    return ((cfg.read_budget_mode in ("absolute", "adaptive_score") and (cfg.read_abs_k > 0 or cfg.read_abs_v > 0))
            or cfg.read_budget_ratio > 0 or (cfg.read_budget_ratio_k or 0) > 0
            or (cfg.read_budget_ratio_v or 0) > 0)
