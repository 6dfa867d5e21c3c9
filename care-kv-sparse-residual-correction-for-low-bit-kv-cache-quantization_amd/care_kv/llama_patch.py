"""HuggingFace LLaMA monkey-patch (llama_patch.py of the reference).

``patch_llama_model(model, care_cfg)`` swaps every attention module that has
a ``q_proj`` for a ``CAREKVLlamaAttention`` running ``CAREKVLayer`` prefill
and decode over one shared ``CAREKVCache`` (all layers, one slot per batch
row).  Differences from the reference, all at the boundary:

* a batch of B > 1 rows runs as one batched kernel call per layer instead of
  a Python loop over per-sequence caches (llama_patch.py:229-258), and a new
  prefill resets the batch's pages for every B (the reference never resets
  for B > 1, its quirk (vi));
* the forward accepts both the transformers 4.x keyword ``past_key_value``
  and the 5.x ``past_key_values``, and returns ``(attn_output, None)`` on
  5.x (``LlamaDecoderLayer`` unpacks two values) and the reference's
  3-tuple on 4.x;
* on transformers 5.x the patched model's own cache is a
  ``CAREKVHFCache``: an HF ``Cache`` whose layers hold only the token count
  HF reads (the rows live in the CARE-KV arena it exposes as
  ``care_cache``), instead of the reference's DynamicCache of fp16 zeros
  (llama_patch.py:262-285, a second KV cache's worth of memory).  A cache
  the caller passes in is kept and fed one-wide placeholders.
"""
from __future__ import annotations

import os
from typing import Dict, Optional

import torch
from torch import nn

from .cache import CAREKVCache
from .config import CacheConfig
from .layer import CAREKVLayer

try:
    import transformers
    _HF_MAJOR = int(transformers.__version__.split(".")[0])
except Exception:  # pragma: no cover
    _HF_MAJOR = 5


if _HF_MAJOR >= 5:
    from transformers.cache_utils import Cache, CacheLayerMixin, DynamicCache

    class _CareLengthLayer(CacheLayerMixin):
        """One layer of ``CAREKVHFCache``: the number of tokens the layer's
        CARE-KV pages hold, which is all HF reads from a cache layer
        (sequence length, mask sizes)."""

        is_sliding = False
        is_compileable = False

        def __init__(self):
            super().__init__()
            self.length = 0

        def lazy_initialization(self, key_states, value_states):
            self.dtype, self.device = key_states.dtype, key_states.device
            self.is_initialized = True

        def update(self, key_states, value_states, *args, **kwargs):
            """Counts the rows; the states themselves go to the CARE-KV pages."""
            if not self.is_initialized:
                self.lazy_initialization(key_states, value_states)
            self.length += key_states.shape[-2]
            return key_states, value_states

        def get_mask_sizes(self, query_length: int):
            return self.length + query_length, 0

        def get_seq_length(self) -> int:
            return self.length

        def get_max_length(self) -> int:
            return -1

        def reset(self):
            self.length = 0

        def offload(self):
            pass

        def prefetch(self):
            pass

        def _unsupported(self, *args, **kwargs):
            raise NotImplementedError("CAREKVHFCache does not crop, reorder or repeat rows (no beam search, "
                                      "no assisted decoding): the pages are append-only")

        crop = reorder_cache = batch_repeat_interleave = batch_select_indices = _unsupported

    class CAREKVHFCache(Cache):
        """The HF ``Cache`` of a patched model: per-layer token counts over
        the CARE-KV cache the patched attention modules share (no fp16 K/V
        copy, llama_patch.py:262-285).  ``care_cache`` is that
        ``CAREKVCache``."""

        def __init__(self, shared: Optional["_SharedState"] = None):
            super().__init__(layer_class_to_replicate=_CareLengthLayer)
            self._shared = shared

        @property
        def care_cache(self):
            return None if self._shared is None else self._shared.cache

        def advance(self, layer_idx: int, n_tokens: int):
            """Record n_tokens new rows of layer ``layer_idx``."""
            while len(self.layers) <= layer_idx:
                self.layers.append(_CareLengthLayer())
            self.layers[layer_idx].length += int(n_tokens)
else:  # pragma: no cover - transformers 4.x keeps the one-wide placeholders
    CAREKVHFCache = None


class _SharedState:
    """One cache for all patched layers of a model and the per-row prefill
    flags of each layer (llama_patch.py:84-101, 321-348)."""

    def __init__(self):
        self.cache: Optional[CAREKVCache] = None
        self.prefilled: Dict[int, set] = {}


class CAREKVLlamaAttention(nn.Module):
    """Wraps a HF ``LlamaAttention`` (llama_patch.py:41-288)."""

    def __init__(self, original_attn: nn.Module, cfg: CacheConfig, layer_id: int, device: torch.device,
                 shared: Optional[_SharedState] = None):
        super().__init__()
        self.cfg = cfg
        self.layer_id = layer_id
        self.device = torch.device(device)
        self.original_attn = original_attn
        self.care_layer = CAREKVLayer(cfg, layer_id, original_attn.q_proj.weight.data,
                                      original_attn.k_proj.weight.data, original_attn.v_proj.weight.data,
                                      original_attn.o_proj.weight.data, device=self.device)
        self._shared = shared if shared is not None else _SharedState()

    # ------------------------------------------------------------ cache
    def _cache_for(self, batch: int, device) -> CAREKVCache:
        st = self._shared
        if st.cache is None or st.cache.n_seq < batch or st.cache.device != torch.device(device):
            # the streaming fill store (no reference counterpart) is on unless
            # cfg.compat; CAREKV_STREAMING_STORE=1 / 0 forces it on / off
            env = os.environ.get("CAREKV_STREAMING_STORE", "")
            st.cache = CAREKVCache(self.cfg, device=device, n_seq=batch,
                                   streaming_store=None if env == "" else env == "1")
            st.prefilled.clear()
        return st.cache

    def reset_cache(self, seq_id: Optional[int] = None):
        """llama_patch.py:103-110: forget every row (or one)."""
        st = self._shared
        if st.cache is None:
            return
        if seq_id is None:
            for s in range(st.cache.n_seq):
                st.cache.reset_sequence(s)
            st.prefilled.clear()
        else:
            st.cache.reset_sequence(seq_id)
            for flags in st.prefilled.values():
                flags.discard(seq_id)

    def _flags(self) -> set:
        return self._shared.prefilled.setdefault(self.layer_id, set())

    # ------------------------------------------------------------ forward
    def forward(self, hidden_states, attention_mask=None, position_ids=None, past_key_value=None,
                output_attentions=False, use_cache=False, cache_position=None, past_key_values=None, **kwargs):
        """llama_patch.py:112-288."""
        pkv = past_key_values if past_key_values is not None else past_key_value
        return_mode = os.environ.get("CAREKV_RETURN", "care").lower()
        position_embeddings = kwargs.get("position_embeddings", None)
        if return_mode in {"original", "passthrough", "hf"} or position_embeddings is None:
            # the reference falls back to HF attention without RoPE inputs
            call = dict(attention_mask=attention_mask, position_ids=position_ids, **kwargs)
            if _HF_MAJOR >= 5:
                call["past_key_values"] = pkv
            else:
                call.update(past_key_value=pkv, output_attentions=output_attentions, use_cache=use_cache)
            if cache_position is not None:
                call["cache_position"] = cache_position
            return self.original_attn(hidden_states, **call)

        B, T, _ = hidden_states.shape
        seqs = list(range(B))
        hf_len = 0
        if use_cache and pkv is not None:
            try:
                hf_len = pkv.get_seq_length(self.layer_id)
            except Exception:
                try:
                    hf_len = pkv.get_seq_length()
                except Exception:
                    hf_len = 0
        cache = self._cache_for(B, hidden_states.device)
        flags = self._flags()
        # a new prompt: several tokens, or one token HF has no cache for
        # (llama_patch.py:177-199); layer 0 clears the rows for every layer
        new_prompt = T > 1 or (use_cache and hf_len == 0 and not all(s in flags for s in seqs))
        if new_prompt:
            if self.layer_id == 0:
                self.reset_cache()
                flags = self._flags()
            flags.difference_update(seqs)
        if not all(s in flags for s in seqs):
            out = self.care_layer.prefill(cache, hidden_states, attention_mask=attention_mask,
                                          position_embeddings=position_embeddings, seqs=seqs)
            flags.update(seqs)
        else:
            out = self.care_layer.decode_step(cache, hidden_states, position_embeddings=position_embeddings,
                                              seqs=seqs)

        # keep HF's own cache length in step so that it sends one token per
        # decode call (llama_patch.py:262-285).  The reference appends fp16
        # zeros of the full K/V shape (a second KV cache's worth of memory).
        # A CAREKVHFCache just counts the rows; a cache the caller passed
        # gets placeholders of head_dim 1: the length HF reads (shape[-2],
        # of a non-empty tensor) advances at 1/head_dim of the memory.
        if use_cache and CAREKVHFCache is not None and isinstance(pkv, CAREKVHFCache):
            pkv.advance(self.layer_id, T)
        elif use_cache and pkv is not None and hasattr(pkv, "update"):
            try:
                z = hidden_states.new_zeros((B, self.cfg.num_kv_heads, T, 1))
                pkv.update(z, z, self.layer_id)
            except Exception:
                pass
        if _HF_MAJOR >= 5:
            return out, None
        return out, None, pkv


def patch_llama_model(model: nn.Module, care_cfg: CacheConfig, device: Optional[torch.device] = None) -> nn.Module:
    """llama_patch.py:292-352: replace every ``*Attention`` module with a
    ``q_proj`` by ``CAREKVLlamaAttention`` (layer id = first integer in the
    module path); all of them share one cache."""
    if device is None:
        try:
            device = next(model.parameters()).device
        except StopIteration:
            device = torch.device("cuda", torch.cuda.current_device())
    shared = _SharedState()
    targets = []
    for name, module in model.named_modules():
        if "Attention" in type(module).__name__ and hasattr(module, "q_proj"):
            targets.append((name, module))
    for name, module in targets:
        parts = name.split(".")
        parent = model
        for part in parts[:-1]:
            parent = getattr(parent, part)
        layer_id = next((int(p) for p in parts if p.isdigit()), 0)
        setattr(parent, parts[-1], CAREKVLlamaAttention(module, care_cfg, layer_id, device, shared=shared))
    if CAREKVHFCache is not None and targets:
        _install_hf_cache(model, shared)
    print(f"[CARE-KV] Replaced {len(targets)} attention layers with CARE-KV.")
    return model


def _install_hf_cache(model: nn.Module, shared: _SharedState):
    """Make ``CAREKVHFCache`` the cache the patched model makes for itself:
    ``generate``'s default DynamicCache (``_prepare_cache_for_generation``)
    and the one the decoder stack creates when called with use_cache and no
    cache.  Caches the caller passes in are left alone."""
    prep = getattr(model, "_prepare_cache_for_generation", None)
    if prep is not None:
        def prepare(*args, **kwargs):
            model_kwargs = kwargs["model_kwargs"] if "model_kwargs" in kwargs else args[1]
            given = model_kwargs.get("past_key_values")
            out = prep(*args, **kwargs)
            made = model_kwargs.get("past_key_values")
            if given is None and type(made) is DynamicCache:
                model_kwargs["past_key_values"] = CAREKVHFCache(shared)
            return out
        model._prepare_cache_for_generation = prepare
    decoder = getattr(model, "model", None)
    if isinstance(decoder, nn.Module) and hasattr(decoder, "layers"):
        cfg_use_cache = bool(getattr(getattr(decoder, "config", None), "use_cache", False))

        def pre_hook(module, args, kwargs):
            use = kwargs.get("use_cache")
            if kwargs.get("past_key_values") is None and (use if use is not None else cfg_use_cache):
                kwargs["past_key_values"] = CAREKVHFCache(shared)
            return args, kwargs
        decoder.register_forward_pre_hook(pre_hook, with_kwargs=True)


def reset_all_caches(model: nn.Module):
    """llama_patch.py:355-359."""
    for module in model.modules():
        if isinstance(module, CAREKVLlamaAttention):
            module.reset_cache()
