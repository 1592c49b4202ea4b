"""Rotary position embedding with the reference's interface.

Drop-in for ``kernels/rope_kernel.py`` and ``ops/rope.py`` of the reference
engine:

* :func:`rope_triton` -- ``kernels/rope_kernel.py:261-285`` (and
  ``_check_cos_sin`` / ``_apply_qk``, 167-258): Q and K rotated in one HIP
  launch (``sia_rope_qk``), strided Q/K slices of a fused qkv buffer read
  without a copy, contiguous outputs.
* :func:`apply_rope` -- ``ops/rope.py:206-226``: the split-half rotation the
  attention module calls.
* :class:`RopeFrequencies` -- ``ops/rope.py:72-185``: the cos/sin tables
  (Llama 3 frequency scaling) and their per-dtype cast cache.

The rotation is ``out_a = x_a cos - x_b sin``, ``out_b = x_b cos + x_a sin``
in fp32 with every product and sum rounded on its own (no fused
multiply-add), stored in the input dtype with round-to-nearest-even.  Row
``r`` of the flattened ``(B*T)`` rows takes position ``r % cos.shape[0]``,
as in the reference kernel.
"""

from __future__ import annotations

import math

import torch

from . import _lib


def _check_cos_sin(cos: torch.Tensor, sin: torch.Tensor, head_dim: int) -> int:
    """The reference's table checks (``kernels/rope_kernel.py:167-190``); returns the row stride."""
    half = head_dim // 2
    if cos.shape[-1] not in (head_dim, half):
        raise ValueError(f"cos/sin last dim must be head_dim ({head_dim}) or head_dim/2 ({half}); "
                         f"got {cos.shape[-1]}")
    if cos.shape != sin.shape:
        raise ValueError(f"cos and sin must have identical shape; got {cos.shape} vs {sin.shape}")
    if cos.stride(-1) != 1 or sin.stride(-1) != 1:
        raise ValueError("cos/sin must be unit-stride along the last dim")
    if cos.stride(0) != sin.stride(0):
        raise ValueError("cos and sin must share the same row stride")
    if cos.dim() != 2:
        raise ValueError(f"cos/sin must be (seq_len, width) tables; got {cos.dim()} dims")
    return cos.stride(0)


def rope_triton(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                interleaved: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate ``q (B, T, Hq, D)`` and ``k (B, T, Hkv, D)`` by the ``cos``/``sin`` tables.

    ``cos``/``sin``: ``(T', D)`` duplicated or ``(T', D/2)`` raw; only the
    first ``D/2`` columns are read.  ``interleaved=False`` pairs ``(i, i+D/2)``
    (Llama/NeoX), ``True`` pairs ``(2i, 2i+1)`` (GPT-J).  Returns contiguous
    ``(q_rot, k_rot)`` with the inputs' shapes and dtypes.
    """
    B, T, n_heads_q, head_dim = q.shape
    _check_cos_sin(cos, sin, head_dim)
    if head_dim % 2:
        raise AssertionError("head_dim must be even for RoPE")
    ks = k.shape
    if ks[0] != B or ks[1] != T or ks[3] != head_dim:
        raise AssertionError(f"k {tuple(ks)} does not match q {tuple(q.shape)} in B, T or head_dim")
    # views whose B*T rows are not one stride apart (head_dim unit-stride,
    # heads head_dim apart, stride(0) == T*stride(1) unless T == 1 or B == 1)
    # are copied by the extension op, which also allocates the outputs
    return _lib.gpu_ops().rope_qk(q, k, cos, sin, bool(interleaved))


def apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """``ops/rope.py:206``: split-half RoPE of ``q``/``k`` with ``(T, head_dim)`` tables."""
    return rope_triton(q, k, cos, sin)


class RopeFrequencies:
    """cos/sin tables for positions ``[0, max_seq_len)`` (``ops/rope.py:72-185``).

    Frequencies ``1 / theta^(2i/D)`` in fp32; with ``rope_type="llama3"`` each
    is rescaled by wavelength (kept below ``original_max_seq_len /
    high_freq_factor``, divided by ``factor`` above ``original_max_seq_len /
    low_freq_factor``, linearly blended between), the blend evaluated in
    double precision as the reference does, then stored as fp32.  Tables are
    fp32 ``(max_seq_len, head_dim)`` with each angle duplicated across the
    two halves.
    """

    def __init__(self, head_dim: int, max_seq_len: int, rope_theta: float = 500_000.0, rope_type: str = "llama3",
                 factor: float = 32.0, low_freq_factor: float = 1.0, high_freq_factor: float = 4.0,
                 original_max_seq_len: int = 8192, device: torch.device | None = None):
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        device = device or torch.device("cuda" if torch.cuda.is_available() else "cpu")
        exponent = torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim
        freqs = 1.0 / (rope_theta ** exponent)
        if rope_type == "llama3":
            freqs = self._llama3_scaled(freqs, factor, low_freq_factor, high_freq_factor, original_max_seq_len)
        angle = torch.outer(torch.arange(max_seq_len, dtype=torch.float32, device=device), freqs)
        angle = torch.cat([angle, angle], dim=-1)
        self.cos = angle.cos()
        self.sin = angle.sin()
        self._cast_cache: dict[torch.dtype, tuple[torch.Tensor, torch.Tensor]] = {}

    @staticmethod
    def _llama3_scaled(freqs: torch.Tensor, factor: float, low_freq_factor: float, high_freq_factor: float,
                       original_max_seq_len: int) -> torch.Tensor:
        f = freqs.double()
        wavelen = (2 * math.pi) / f
        smooth = (original_max_seq_len / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
        blended = (1 - smooth) * f / factor + smooth * f
        out = torch.where(wavelen > original_max_seq_len / low_freq_factor, f / factor, blended)
        out = torch.where(wavelen < original_max_seq_len / high_freq_factor, f, out)
        return out.to(freqs.dtype)

    def get(self, seq_len: int, start_pos: int = 0, dtype: torch.dtype | None = None):
        """``(cos, sin)`` rows ``[start_pos, start_pos + seq_len)``, cast to ``dtype`` from a cached full table."""
        if dtype is None or dtype == torch.float32:
            cos_tbl, sin_tbl = self.cos, self.sin
        else:
            cached = self._cast_cache.get(dtype)
            if cached is None:
                cached = (self.cos.to(dtype), self.sin.to(dtype))
                self._cast_cache[dtype] = cached
            cos_tbl, sin_tbl = cached
        return cos_tbl[start_pos:start_pos + seq_len], sin_tbl[start_pos:start_pos + seq_len]
