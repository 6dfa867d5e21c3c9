"""``CAREKVAdapter`` (baselines/carekv_adapter.py:15-263 of the reference):
the evaluation-harness entry point that configures CARE-KV through the
``CAREKV_*`` environment and patches a LLaMA model.

Same constructor, ``setup_model`` environment and reporting methods, with
the fixed (RK/RV) and the adaptive (adaptive_score with rel_threshold under
the max_rk/max_rv caps) read budgets.  The uniform packed base and the
side-buffer bases kivi_style / kvquant_style (post-RoPE) are built; the
rotation bases (RotateKV, random rotation) and pre-RoPE KVQuant raise
``NotImplementedError``.  ``setup_model`` also accepts an already built
``nn.Module`` (a random-init model when no checkpoint is at hand)."""
from __future__ import annotations

import os
from typing import Union

import torch
from torch import nn

from .config import CacheConfig, apply_carekv_env_overrides
from .llama_patch import CAREKVLlamaAttention, patch_llama_model, reset_all_caches


def fp16_kv_mb(seq_len: int, num_layers: int = 22, hkv: int = 4, head_dim: int = 64) -> float:
    """baselines/common.py:143-145."""
    return num_layers * 2 * seq_len * hkv * head_dim * 2 / (1024 * 1024)


class CAREKVAdapter:
    family = "care_kv"
    is_official = False
    is_reimplementation = True
    uses_residual = True
    uses_query_aware_routing = True

    def __init__(self, mode: str = "fixed", rel_threshold: float = 0.0, sk: int = 2, sv: int = 4, rk: int = 2,
                 rv: int = 2, max_rk: int = 4, max_rv: int = 4, bits: int = 3, base_quantizer: str = "uniform",
                 bits_k: int = -1, bits_v: int = -1, max_pages: int = 0, k_store_mode: str = "post_rope",
                 correction_impl: str = "cached", k_channel_group: int = 32, v_token_block: int = 4):
        if base_quantizer not in ("uniform", "kivi_style", "kvquant_style"):
            raise NotImplementedError(f"base_quantizer={base_quantizer!r}: the uniform, kivi_style and "
                                      "kvquant_style (post-RoPE) bases are built")
        if base_quantizer == "kvquant_style" and k_store_mode != "post_rope":
            raise NotImplementedError("kvquant_style with k_store_mode=pre_rope is not built")
        if mode not in ("fixed", "adaptive"):
            raise ValueError(f"mode must be 'fixed' or 'adaptive' (got {mode!r})")
        self.mode, self.rel_threshold = mode, rel_threshold
        self.sk, self.sv, self.rk, self.rv = sk, sv, rk, rv
        self.max_rk, self.max_rv = max_rk, max_rv
        self.bits = bits
        self.base_quantizer = base_quantizer
        self.k_store_mode = k_store_mode
        self.correction_impl = correction_impl
        self.k_channel_group, self.v_token_block = k_channel_group, v_token_block
        self.bits_k = bits_k if bits_k > 0 else bits
        self.bits_v = bits_v if bits_v > 0 else bits
        self.max_pages = max_pages if max_pages > 0 else 512
        self.name = (f"CAREKV_adaptive_rel{rel_threshold:.2f}" if mode == "adaptive"
                     else f"CAREKV_fixed_SK{sk}SV{sv}_RK{rk}RV{rv}")
        self.bit_width = f"INT{bits}"
        self.k_quant_scheme = "per-channel-group=32 + selected residual slots"
        self.v_quant_scheme = "per-channel-group=32 + selected residual slots"
        self.model = None

    def env(self) -> dict:
        """The CAREKV_* settings of setup_model (carekv_adapter.py:103-145)."""
        read = (dict(CAREKV_READ_BUDGET_MODE="adaptive_score", CAREKV_READ_ABS_K=str(self.max_rk),
                     CAREKV_READ_ABS_V=str(self.max_rv), CAREKV_READ_RELATIVE_THRESHOLD=str(self.rel_threshold))
                if self.mode == "adaptive" else
                dict(CAREKV_READ_BUDGET_MODE="absolute", CAREKV_READ_ABS_K=str(self.rk),
                     CAREKV_READ_ABS_V=str(self.rv), CAREKV_READ_RELATIVE_THRESHOLD="0.0"))
        return dict(**read,
            CAREKV_PREFILL_MODE="carekv_stored", CAREKV_PREFILL_RESIDUAL_KIND="both", CAREKV_ROUTE_POLICY="joint",
            CAREKV_SCORE_NORMALIZE="1", CAREKV_CORRECTION_IMPL=self.correction_impl, CAREKV_BUDGET_POLICY="uniform",
            CAREKV_PACKED_BASE="1", CAREKV_SCALE_QUANT="int8", CAREKV_BASE_BITS=str(self.bits),
            CAREKV_GROUP_SIZE="32", CAREKV_STORE_BUDGET_MODE="absolute", CAREKV_STORE_ABS_K=str(self.sk),
            CAREKV_STORE_ABS_V=str(self.sv), CAREKV_DEBUG_STATS="1", CAREKV_BASE_QUANTIZER=self.base_quantizer,
            CAREKV_K_BITS=str(self.bits_k), CAREKV_V_BITS=str(self.bits_v), CAREKV_K_STORE_MODE=self.k_store_mode,
            CAREKV_K_CHANNEL_GROUP=str(self.k_channel_group), CAREKV_V_TOKEN_BLOCK=str(self.v_token_block),
            CAREKV_READ_ABSOLUTE_THRESHOLD="0.0", CAREKV_READ_MIN_KEEP="0")

    def setup_model(self, model_id: Union[str, nn.Module]):
        """carekv_adapter.py:101-172: set the environment, load (a local
        checkpoint path, fp16) or take the given model, patch it."""
        from .attention import reset_debug_stats
        reset_debug_stats()
        for k, v in self.env().items():
            os.environ[k] = v
        torch.manual_seed(0)
        if isinstance(model_id, nn.Module):
            m = model_id
        else:
            from transformers import LlamaForCausalLM
            m = LlamaForCausalLM.from_pretrained(model_id, torch_dtype=torch.float16, low_cpu_mem_usage=True)
            m = m.to(torch.device("cuda", torch.cuda.current_device()))
        m.config.use_cache = False
        c = m.config
        hd = getattr(c, "head_dim", None) or c.hidden_size // c.num_attention_heads
        kw = dict(num_layers=c.num_hidden_layers, num_heads=c.num_attention_heads,
                  num_kv_heads=c.num_key_value_heads, head_dim=hd, base_bits=self.bits, group_size=32,
                  k_channel_group=32, page_size=16, max_pages=self.max_pages, v_token_block=4, sketch_dim=32,
                  store_budget_ratio=0.0, read_budget_ratio=0.0, store_budget_mode="absolute",
                  read_budget_mode="absolute")
        apply_carekv_env_overrides(kw)
        m = patch_llama_model(m, CacheConfig(**kw))
        reset_all_caches(m)
        m.eval()
        self.model = m
        return m

    def collect_debug_stats(self):
        """carekv_adapter.py:174-181: the K / V slots the correction read
        (device counters, CAREKV_DEBUG_STATS=1 as setup_model sets it) and the
        slots the store holds."""
        from .attention import get_debug_stats
        st = get_debug_stats()
        sk = sv = 0
        if self.model is not None:
            for mod in self.model.modules():
                if isinstance(mod, CAREKVLlamaAttention) and mod._shared.cache is not None:
                    cache = mod._shared.cache
                    for s in range(cache.n_seq):
                        k, v = cache.num_stored_residual_slots(s)
                        sk += k
                        sv += v
                    break
        return dict(k_reads=int(st["k_slots_read"]), v_reads=int(st["v_slots_read"]), stored_k_slots=int(sk),
                    stored_v_slots=int(sv))

    def estimate_memory(self, seq_len: int, num_layers: int = 22, hkv: int = 4, head_dim: int = 64):
        """carekv_adapter.py:183-223, uniform base."""
        fp16 = fp16_kv_mb(seq_len, num_layers, hkv, head_dim)
        base_mb = fp16 * (self.bits / 16.0)
        residual_mb = fp16 * 0.05
        total = base_mb + residual_mb
        return dict(estimated_kv_memory_MB=round(total, 4), estimated_total_cache_memory_MB=round(total, 4),
                    vs_fp16_kv_memory_ratio=round(total / max(fp16, 1e-9), 4), base_memory_MB=round(base_mb, 4),
                    residual_memory_MB=round(residual_mb, 4), base_quantizer=self.base_quantizer)

    def effective_budgets(self):
        read = (f"adaptive rel={self.rel_threshold} max RK={self.max_rk} RV={self.max_rv}"
                if self.mode == "adaptive" else f"fixed RK={self.rk} RV={self.rv}")
        return dict(effective_store_budget=f"SK={self.sk} SV={self.sv}", effective_read_budget=read)

    def notes(self) -> str:
        return ("CARE-KV paper-best (carekv_stored, joint+normalize, cached, "
                f"SK={self.sk} SV={self.sv} RK={self.rk} RV={self.rv}).")
