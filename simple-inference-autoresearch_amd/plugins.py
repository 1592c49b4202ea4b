"""Model-plugin hooks: cache builders and the transformers attention interface.

* :func:`llama_cache_builder` -- drop-in for the llama plugin's
  ``cache_builder`` (``model/llama_plugin.py:22-38``): same keyword
  arguments, returns this library's :class:`~.kv_cache.KVCache` (int8 pools
  once ``max_seq_len`` exceeds the reference's threshold).
  :func:`llama_paged_cache_builder` builds a :class:`~.paged_kv_cache.PagedKVCache`
  with the same arguments (plus ``block_size`` / ``kv_dtype``).
* :func:`sia_attention_forward` -- an attention function with the
  transformers attention-interface contract that the Qwen3.5 full-attention
  layers call through ``ALL_ATTENTION_FUNCTIONS.get_interface(
  config._attn_implementation)`` (``model/qwen35_plugin.py:396-402``;
  transformers ``Qwen3_5Attention.forward``): ``(module, query (B, Hq, T, D),
  key, value (B, Hkv, S, D), attention_mask, dropout=, scaling=, **kwargs)``
  -> ``(attn_output (B, T, Hq, D), None)``.  The caller applies its output
  gate (``* sigmoid(gate)``) and ``o_proj`` afterwards, as with any backend.
  :func:`register_attention` registers it (and a matching mask builder) under
  a name; :func:`use_for` points a model config at it.

transformers is imported only when registering (it is a dependency of the
reference's Qwen plugin, not of this library's kernels).
"""

from __future__ import annotations

import torch

from .kv_cache import KVCache
from .paged_kv_cache import PagedKVCache
from .prefill import attention_flash_triton

ATTENTION_NAME = "sia"


# ------------------------------------------------------------ cache builders


def llama_cache_builder(config, *, max_batch: int, max_seq_len: int, dtype: torch.dtype,
                        device: torch.device | str) -> KVCache:
    """The llama plugin's cache hook (``model/llama_plugin.py:22-38``) on this library's KVCache."""
    return KVCache(n_layers=config.num_hidden_layers, max_batch=max_batch, max_seq_len=max_seq_len,
                   n_heads_kv=config.num_key_value_heads, head_dim=config.head_dim, dtype=dtype, device=device)


def llama_paged_cache_builder(config, *, max_batch: int, max_seq_len: int, dtype: torch.dtype,
                              device: torch.device | str, block_size: int = 16,
                              kv_dtype: torch.dtype | None = None) -> PagedKVCache:
    """Same hook, building a paged cache (``kv_dtype=torch.int8`` for int8 pools with fp32 scales)."""
    return PagedKVCache(config.num_hidden_layers, max_batch, max_seq_len, config.num_key_value_heads,
                        config.head_dim, block_size=block_size, dtype=dtype, device=device, kv_dtype=kv_dtype)


# ------------------------------------------------ transformers attention hook


def _padding_free(attention_mask) -> bool:
    """True when the model passes no mask: the un-padded case.

    The mask builder registered with this function (transformers'
    ``flash_attention_2`` one) already returns ``None`` for a batch without
    padding, once per forward; any mask it does return marks padded keys (or
    a static cache's unfilled slots), which no kernel here handles.  So the
    decision needs no look at the mask's values: no device-to-host copy per
    layer, and a decode step stays capturable in a HIP graph.  The
    reference's Qwen3.5 plugin calls the backbone without a mask
    (``model/qwen35_plugin.py:396-402``), which is the ``None`` case.
    """
    return attention_mask is None


def sia_attention_forward(module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, attention_mask,
                          dropout: float = 0.0, scaling: float | None = None, is_causal: bool | None = None,
                          **kwargs):
    """transformers attention-interface function backed by the gfx950 kernels.

    Causal (bottom-right aligned, so a query block at the end of a cached
    prefix sees the whole prefix) when the module is causal, full otherwise.
    GQA is resolved by head index, with no ``repeat_kv`` copy.  Padding masks,
    dropout, sliding windows and soft-capping have no kernel here and raise
    ``NotImplementedError`` rather than being ignored.
    """
    if dropout:
        raise NotImplementedError("attention dropout is not supported by the gfx950 kernels")
    if kwargs.get("sliding_window") is not None or kwargs.get("softcap") is not None:
        raise NotImplementedError("sliding-window / soft-capped attention is not supported")
    if not _padding_free(attention_mask):
        raise NotImplementedError("an attention mask (padded batch or static-cache slots) is not supported; "
                                  "un-padded batches reach this function with attention_mask=None")
    causal = getattr(module, "is_causal", True) if is_causal is None else bool(is_causal)
    out = attention_flash_triton(query, key, value, causal=causal, sm_scale=scaling, out_token_major=True)
    return out, None


def register_attention(name: str = ATTENTION_NAME) -> str:
    """Register :func:`sia_attention_forward` (and an un-padded mask builder) with transformers."""
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, AttentionMaskInterface

    AttentionInterface.register(name, sia_attention_forward)
    # the model then passes None (no padding) or the 2D padding mask, as for
    # the un-padded flash-attention backends
    AttentionMaskInterface.register(name, ALL_MASK_ATTENTION_FUNCTIONS["flash_attention_2"])
    return name


def use_for(config, name: str = ATTENTION_NAME):
    """Select the registered kernels for every attention layer built from ``config``."""
    register_attention(name)
    config._attn_implementation = name
    return config
