"""Prefill / general attention with the reference's signature.

``attention_flash_triton`` is a drop-in for the reference function of the same
name (kernels/attention_kernel.py:235-305): same arguments, same output layout
and dtype, same causal convention (query row i sits at position (Tk - Tq) + i)
and the same assertion on head_dim.  It runs the gfx950 MFMA kernel behind
``sia_attention_flash_fwd``; there is no Triton involved despite the name,
which is kept so callers need no change.
"""

from __future__ import annotations

import functools

import torch

from . import _lib

_HEAD_DIMS = (16, 32, 64, 128, 256)
_DECODE_DIMS = (64, 128, 256)   # head dims of the decode kernels (single-query calls)


@functools.lru_cache(maxsize=256)
def prefill_workspace_size(batch: int, kv_heads: int, kv_len: int, head_dim: int) -> int:
    """Bytes of device workspace ``sia_attention_flash_fwd`` needs (f16 V^T block images)."""
    return int(_lib.gpu_ops().prefill_workspace_size(batch, kv_heads, kv_len, head_dim))


_OPS = None   # the extension module, once loaded on a GPU


def _ops():
    global _OPS
    if _OPS is None:
        _OPS = _lib.gpu_ops()
    return _OPS


def attention_flash_triton(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool,
                           sm_scale: float | None = None, assume_contiguous: bool = False,
                           out_token_major: bool = False) -> torch.Tensor:
    """Flash-attention forward.

    q: (B, Hq, Tq, D); k, v: (B, Hkv, Tk, D); returns (B, Hq, Tq, D), or
    (B, Tq, Hq, D) when ``out_token_major``, in q's dtype.  Strided views are
    read in place; the extension copies a view only when its layout cannot be
    read directly (head_dim not contiguous, rows not 16-byte aligned, or rows
    too far apart for 32-bit offsets within a 64-key block), so
    ``assume_contiguous`` never changes the result.
    """
    B, Hq, Tq, D = q.shape
    _, Hkv, Tk, _ = k.shape
    if not (k.shape[-1] == D and v.shape[-1] == D):
        raise AssertionError()
    if D not in _HEAD_DIMS:
        raise AssertionError(f"unsupported head_dim {D}")
    if sm_scale is None:
        sm_scale = 1.0 / (D ** 0.5)
    ops = _ops()
    if Tq == 1 and Tk >= 1 and D in _DECODE_DIMS and k.dtype == q.dtype and v.dtype == q.dtype and q.is_cuda:
        # one query row sees every key (bottom-right causal == full at Tq = 1):
        # the decode kernels stream K/V once per KV-head group instead of
        # occupying a 256-row prefill work-group per head
        from .decode import CONTIG, _run
        kv_len = torch.full((1,), Tk, dtype=torch.int32, device=q.device)
        out = _run(CONTIG, q, k, v, None, None, None, kv_len, 0, float(sm_scale))
        return out if out_token_major else out.view(B, Hq, 1, D)
    return ops.prefill(q, k, v, bool(causal), float(sm_scale), bool(out_token_major))


def rope_attention_flash_triton(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                                sin: torch.Tensor, causal: bool, sm_scale: float | None = None,
                                start_pos: torch.Tensor | None = None, start_offset: int = 0,
                                interleaved: bool = False, out_token_major: bool = False) -> torch.Tensor:
    """``attention_flash_triton(rope(q), k, v)`` in one launch (``sia_attention_flash_fwd_rope``).

    The pair the reference's prefill runs -- ``apply_rope`` on q
    (``ops/attention.py:291-292``, ``kernels/rope_kernel.py:261``) then
    ``attention_flash_triton`` (``ops/attention.py:327-330``) -- with q rotated
    in registers as it is loaded, so no rotated copy of q is written or read.
    ``q (B, Hq, Tq, D)`` is un-rotated; ``k`` already holds rotated keys
    (e.g. the cache that :func:`rope_kv_write` with ``q=None`` filled).  Query
    row ``i`` of sequence ``b`` sits at position
    ``start_offset + start_pos[b] + i`` (``start_pos``: int32 device tensor of
    1 or B elements, or None for 0) and is rotated by that row of the full
    ``cos``/``sin`` tables.  The rotation is :func:`rope_triton`'s arithmetic
    and rounding, so the result equals ``rope_triton`` then
    ``attention_flash_triton`` bit for bit.  float16/bfloat16 only.
    """
    B, Hq, Tq, D = q.shape
    if not (k.shape[-1] == D and v.shape[-1] == D):
        raise AssertionError()
    if D not in _HEAD_DIMS:
        raise AssertionError(f"unsupported head_dim {D}")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise NotImplementedError("the fused rotary prologue runs on float16/bfloat16 inputs; "
                                  "use rope_triton then attention_flash_triton for float32")
    if sm_scale is None:
        sm_scale = 1.0 / (D ** 0.5)
    if cos.dtype not in (q.dtype, torch.float32) and cos.dtype in (torch.float16, torch.bfloat16):
        # the kernel reads tables in q's dtype or fp32; widening the other
        # 16-bit type to fp32 is exact, and the rotation runs in fp32 anyway
        cos, sin = cos.float(), sin.float()
    return _ops().prefill_rope(q, k, v, cos, sin, bool(interleaved), start_pos, int(start_offset),
                                       bool(causal), float(sm_scale), bool(out_token_major))
