"""Prefill / general attention with the reference's signature.

``attention_flash_triton`` is a drop-in for the reference function of the same
name (kernels/attention_kernel.py:235-305): same arguments, same output layout
and dtype, same causal convention (query row i sits at position (Tk - Tq) + i)
and the same assertion on head_dim.  It runs the gfx950 MFMA kernel behind
``sia_attention_flash_fwd``; there is no Triton involved despite the name,
which is kept so callers need no change.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_HEAD_DIMS = (16, 32, 64, 128, 256)


def _supported_view(t: torch.Tensor) -> bool:
    if t.stride(-1) != 1 or t.data_ptr() % 16:
        return False
    es = t.element_size()
    return all((s * es) % 16 == 0 for s in t.stride()[:-1])


def attention_flash_triton(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool,
                           sm_scale: float | None = None, assume_contiguous: bool = False,
                           out_token_major: bool = False) -> torch.Tensor:
    """Flash-attention forward.

    q: (B, Hq, Tq, D); k, v: (B, Hkv, Tk, D); returns (B, Hq, Tq, D), or
    (B, Tq, Hq, D) when ``out_token_major``, in q's dtype.  Strided views are
    read in place; a view is copied only when its layout cannot be read
    directly (head_dim not contiguous or rows not 16-byte aligned), so
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
    h = _lib.require_library()
    if not q.is_cuda:
        raise ValueError("attention runs on the GPU: q must be a CUDA (HIP) tensor")
    q, k, v = (t if _supported_view(t) else t.contiguous() for t in (q, k, v))
    with torch.cuda.device(q.device):
        if out_token_major:
            out = torch.empty((B, Tq, Hq, D), dtype=q.dtype, device=q.device)
            out_view = out.transpose(1, 2)
        else:
            out = torch.empty((B, Hq, Tq, D), dtype=q.dtype, device=q.device)
            out_view = out
        dq, dk, dv, do = (_lib.desc(t) for t in (q, k, v, out_view))
        rc = h.sia_attention_flash_fwd(ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv),
                                       ctypes.c_int32(1 if causal else 0), ctypes.c_float(float(sm_scale)),
                                       ctypes.byref(do), ctypes.c_void_p(_lib.stream_handle(q.device)))
        _lib.check(rc)
    return out
