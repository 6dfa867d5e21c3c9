"""CARE-KV quantized decode attention for MI355X (gfx950 HIP kernels).

The public surface follows the reference package's ``__init__`` (same names,
arguments and results): the cache and its configuration, the quantizer and
bit packers, the store-time and read-time residual classes, the attention
and layer classes, the LLaMA patch the debug counters and the analysis utilities; the compute runs
in ``libcarekv_hip.so`` through a C ABI (include/carekv.h).  Additions of
this build: the batched entry points ``decode_attention`` /
``prefill_correction`` / ``prefill_attention``, ``CAREKVAdapter`` and
``CarekvError``.
"""
from .config import (CacheConfig, apply_carekv_env_overrides, layer_budget_multiplier,
                     resolve_read_knobs, resolve_store_knobs)
from .cache import CAREKVCache, PageMeta, get_sketch_proj, kivi_codes, kivi_qdq, packed_row_bytes
from .quantizer import (QuantConfig, KQuantizer, VQuantizer, quantize, dequantize, quantize_and_residual,
                        pack_int2, unpack_int2, pack_int3, unpack_int3, pack_int4, unpack_int4,
                        pack_int2_2d, unpack_int2_2d, pack_int3_2d, unpack_int3_2d, pack_int4_2d, unpack_int4_2d,
                        pack_codes_2d, unpack_codes_2d)
from .residual import ResidualStoreManager, ResidualRouter, pack_4bit, unpack_4bit
from .attention import (CAREKVAttention, CAREKVMultiHeadAttention, apply_slot_corrections, decode_attention,
                        get_debug_stats, prefill_correction, reset_debug_stats)
from .prefill import dequantize_rows, prefill_attention, prefill_eval, quant_dequant, quantize_rows
from .layer import CAREKVLayer
from .attention import get_imp_per_layer
from .utils import (ABLATION_VARIANTS, budget_sweep, calibrate_layer_sensitivity, compute_boundary_risk_stats,
                    compute_perplexity, estimate_memory_bytes, print_memory_table)
from .llama_patch import CAREKVHFCache, CAREKVLlamaAttention, patch_llama_model, reset_all_caches
from .adapter import CAREKVAdapter
from ._lib import CarekvError

__version__ = "0.2.0"
__all__ = [
    "CacheConfig", "CAREKVCache", "PageMeta",
    "apply_carekv_env_overrides", "layer_budget_multiplier",
    "QuantConfig", "KQuantizer", "VQuantizer",
    "quantize", "dequantize", "quantize_and_residual",
    "pack_int2", "unpack_int2", "pack_int3", "unpack_int3",
    "pack_int4", "unpack_int4",
    "pack_int2_2d", "unpack_int2_2d", "pack_int3_2d", "unpack_int3_2d",
    "pack_int4_2d", "unpack_int4_2d",
    "pack_codes_2d", "unpack_codes_2d", "packed_row_bytes",
    "ResidualStoreManager", "pack_4bit", "unpack_4bit",
    "ResidualRouter",
    "CAREKVAttention", "CAREKVMultiHeadAttention", "apply_slot_corrections",
    "CAREKVLayer", "get_debug_stats", "reset_debug_stats", "get_imp_per_layer",
    "CAREKVLlamaAttention", "patch_llama_model", "reset_all_caches",
    "estimate_memory_bytes", "print_memory_table",
    "calibrate_layer_sensitivity", "compute_perplexity",
    "budget_sweep", "compute_boundary_risk_stats",
    "ABLATION_VARIANTS",
    # additions of this build
    "resolve_read_knobs", "resolve_store_knobs", "get_sketch_proj", "kivi_qdq", "kivi_codes",
    "decode_attention", "prefill_correction", "prefill_attention", "prefill_eval", "quantize_rows", "dequantize_rows",
    "quant_dequant", "CAREKVAdapter", "CarekvError", "CAREKVHFCache",
]
