"""CARE-KV quantized decode attention for MI355X (gfx950 HIP kernels).

Public surface follows the reference package's names (``CacheConfig``,
``CAREKVCache``, ``PageMeta``, ``apply_carekv_env_overrides``,
``layer_budget_multiplier``, ``CAREKVMultiHeadAttention``, ...); the compute
runs in ``libcarekv_hip.so`` through a C ABI (include/carekv.h).
"""
from .config import (CacheConfig, apply_carekv_env_overrides, layer_budget_multiplier,
                     resolve_read_knobs, resolve_store_knobs)
from .cache import CAREKVCache, PageMeta, get_sketch_proj, kivi_qdq, packed_row_bytes
from .attention import CAREKVMultiHeadAttention, decode_attention, prefill_correction
from .prefill import dequantize_rows, prefill_attention, quant_dequant, quantize_rows
from .layer import CAREKVLayer
from .llama_patch import CAREKVLlamaAttention, patch_llama_model, reset_all_caches
from .adapter import CAREKVAdapter
from ._lib import CarekvError

__version__ = "0.1.0"
__all__ = [
    "CacheConfig", "apply_carekv_env_overrides", "layer_budget_multiplier", "resolve_read_knobs",
    "resolve_store_knobs", "CAREKVCache", "PageMeta", "get_sketch_proj", "kivi_qdq", "packed_row_bytes",
    "CAREKVMultiHeadAttention", "decode_attention", "prefill_correction", "prefill_attention", "quantize_rows", "dequantize_rows",
    "quant_dequant", "CAREKVLayer", "CAREKVLlamaAttention", "patch_llama_model", "reset_all_caches",
    "CAREKVAdapter", "CarekvError",
]
