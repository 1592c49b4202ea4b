"""The attention steps of ``GroupedQueryAttention`` (``ops/attention.py``) on this library.

The reference's attention module does projections, RoPE, the cache write,
attention and the output projection.  Only the cache write and the attention
belong to this library's path; these functions are the drop-ins for exactly
those lines, so a caller keeps its own projections and RoPE:

* :func:`gqa_attention` -- the attention of the eager forward
  (``ops/attention.py:311-345``): causal for T > 1, full for T == 1, GQA by
  head index (no ``repeat_interleave`` copy), token-major output reshaped to
  ``(B, T, Hq * D)``.
* :func:`decode_step_attention` -- the cache write and attention of the
  captured decode step (``ops/attention.py:206-231``) over a contiguous
  :class:`~.kv_cache.KVCache`: int8 caches quantise the new token on the way
  in, and the position and length are read on the device from ``ctx``.
* :func:`rope_decode_step_attention` -- the same step from the pre-RoPE
  projections (``ops/attention.py:202-231``): RoPE of q and k fused into the
  cache write, then attention.
* :class:`DecodeCtx` -- the device buffers of ``model/cuda_graph_decode.py:53-56``
  (``cos``, ``sin``, ``pos_index``, ``kv_len``), with int32 positions and
  :meth:`DecodeCtx.set_position` for the per-step update
  (``model/cuda_graph_decode.py:98-102``).
"""

from __future__ import annotations

import torch

from .decode import attention_flash_decode, attention_flash_decode_int8
from .kv_cache import KVCache
from .prefill import attention_flash_triton


def gqa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool | None = None) -> torch.Tensor:
    """Attention of ``q (B, Hq, T, D)`` over ``k, v (B, Hkv, S, D)`` -> ``(B, T, Hq * D)``.

    ``causal`` defaults to the reference's rule ``T > 1`` (bottom-right
    aligned, so a query block at the end of a longer cache sees its prefix).
    """
    B, Hq, T, D = q.shape
    if causal is None:
        causal = T > 1
    out = attention_flash_triton(q, k, v, causal=causal, assume_contiguous=True, out_token_major=True)
    return out.view(B, T, Hq * D)


class DecodeCtx:
    """Per-step decode position in device memory (one captured graph serves every step)."""

    __slots__ = ("cos", "sin", "pos_index", "kv_len")

    def __init__(self, head_dim: int, device, dtype=torch.bfloat16, batch: int = 1, per_sequence: bool = False):
        n = batch if per_sequence else 1
        self.cos = torch.zeros(1, head_dim, dtype=dtype, device=device)
        self.sin = torch.zeros(1, head_dim, dtype=dtype, device=device)
        self.pos_index = torch.zeros(n, dtype=torch.int32, device=device)
        self.kv_len = torch.zeros(n, dtype=torch.int32, device=device)

    def set_position(self, pos) -> None:
        """Position of the token being decoded (int, or a (B,) tensor of per-sequence positions)."""
        if isinstance(pos, torch.Tensor):
            self.pos_index.copy_(pos)
            torch.add(self.pos_index, 1, out=self.kv_len)
        else:
            self.pos_index.fill_(int(pos))
            self.kv_len.fill_(int(pos) + 1)


def rope_decode_step_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                               sin: torch.Tensor, kv_cache: KVCache, layer_idx: int, ctx: DecodeCtx,
                               sm_scale: float | None = None, interleaved: bool = False) -> torch.Tensor:
    """RoPE, cache write and attention of one decode step: ``q (B, 1, Hq, D)``, ``k, v (B, 1, Hkv, D)``.

    Replaces ``ops/attention.py:202-231`` (``apply_rope`` through the
    attention call) with two launches: the fused RoPE + K/V write
    (``sia_rope_kv_write``, which also rotates q) and the decode kernels.
    ``q, k, v`` are the projections before RoPE, token-major as
    ``_project_qkv`` returns them; ``cos``/``sin`` are the full tables, read
    at ``ctx.pos_index`` on the device (``ctx.cos``/``ctx.sin`` are not used).
    Returns ``(B, 1, Hq, D)``.  Graph safe.
    """
    q_rot = kv_cache.write_decode_rope(layer_idx, ctx.pos_index, q, k, v, cos, sin, interleaved=interleaved)
    B = q.shape[0]
    kc, vc, ks, vs = kv_cache._layer(layer_idx, B)
    qh = q_rot.transpose(1, 2)
    if kv_cache.is_int8:
        return attention_flash_decode_int8(qh, kc, vc, ks, vs, ctx.kv_len, sm_scale)
    return attention_flash_decode(qh, kc, vc, ctx.kv_len, sm_scale)


def decode_step_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_cache: KVCache, layer_idx: int,
                          ctx: DecodeCtx, sm_scale: float | None = None) -> torch.Tensor:
    """Write this step's K/V and attend: ``q (B, Hq, 1, D)``, ``k, v (B, Hkv, 1, D)`` -> ``(B, 1, Hq, D)``.

    Replaces ``ops/attention.py:210-231``: the token is written at
    ``ctx.pos_index`` (quantised for an int8 cache) and attention covers the
    first ``ctx.kv_len`` cached positions.  Graph safe: every length and
    position is read on the device.
    """
    B = q.shape[0]
    kv_cache.write_decode(layer_idx, ctx.pos_index, k, v)
    kc, vc, ks, vs = kv_cache._layer(layer_idx, B)
    if kv_cache.is_int8:
        return attention_flash_decode_int8(q, kc, vc, ks, vs, ctx.kv_len, sm_scale)
    return attention_flash_decode(q, kc, vc, ctx.kv_len, sm_scale)
