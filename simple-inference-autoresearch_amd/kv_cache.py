"""Contiguous KV cache and the INT8-KV format, with the reference's interface.

Drop-in for ``model/kv_cache.py`` of the reference engine:

* :func:`quantize_kv_int8` -- ``model/kv_cache.py:58-67`` (same arguments,
  outputs and rounding), computed by the gfx950 kernel behind
  ``sia_quantize_kv_int8``.
* :class:`KVCache` -- ``model/kv_cache.py:70-212``: the same pools
  ``(L, B, Hkv, S, D)`` (int8 with fp16 scales once ``max_seq_len`` exceeds
  ``INT8_SEQ_THRESHOLD``), the same ``update`` contract and return values.
  The writes run as one HIP launch (``sia_kv_write``) instead of the
  quantise-then-slice-assign sequence.
* :meth:`KVCache.write_decode` -- the CUDA-graph decode write of
  ``ops/attention.py:217-228`` (``quantize_kv_int8`` + four ``index_copy_`` at
  ``ctx.pos_index``) as one launch that reads the position on the device.

:func:`kv_write` is the general entry point both caches use.
"""

from __future__ import annotations

import torch

from . import _lib


def kv_write(k: torch.Tensor, v: torch.Tensor | None, k_dst: torch.Tensor, v_dst: torch.Tensor | None,
             k_scale_dst: torch.Tensor | None = None, v_scale_dst: torch.Tensor | None = None,
             block_table: torch.Tensor | None = None, start_pos: torch.Tensor | None = None,
             start_offset: int = 0, page_size: int = 0) -> None:
    """Write tokens ``k/v (B, H, T, D)`` into a cache (``sia_kv_write``).

    Token ``t`` of sequence ``b`` goes to position ``start_offset + start_pos[b] + t``
    (``start_pos``: int32 device tensor of 1 or B elements, or None for 0).
    Without ``block_table`` the destinations are contiguous ``(B', H, S, D)``
    views; with it they are paged pools ``(num_pages, H, page_size, D)``.
    An int8 destination is quantised per token and head (scales written to
    ``k_scale_dst`` / ``v_scale_dst``); other destinations receive a cast copy.
    """
    _lib.gpu_ops().kv_write(k, v, k_dst, v_dst, k_scale_dst, v_scale_dst, block_table, start_pos,
                            int(start_offset), int(page_size))


def rope_kv_write(q: torch.Tensor | None, k: torch.Tensor, v: torch.Tensor | None, cos: torch.Tensor,
                  sin: torch.Tensor, k_dst: torch.Tensor, v_dst: torch.Tensor | None,
                  k_scale_dst: torch.Tensor | None = None, v_scale_dst: torch.Tensor | None = None,
                  block_table: torch.Tensor | None = None, start_pos: torch.Tensor | None = None,
                  start_offset: int = 0, page_size: int = 0, interleaved: bool = False,
                  q_out: torch.Tensor | None = None) -> torch.Tensor | None:
    """RoPE-K fused into the cache write, q rotated in the same launch (``sia_rope_kv_write``).

    ``q (B, T, Hq, D)``, ``k, v (B, T, Hkv, D)``: token-major, as the qkv
    projection leaves them (strided slices are read in place).  Token ``t`` of
    sequence ``b`` sits at position ``p = start_offset + start_pos[b] + t`` and
    is rotated by row ``p`` of the full ``cos``/``sin`` tables.  The rotated K
    (rounded to k's dtype) and V are written like :func:`kv_write` writes them;
    the rotated q is returned as ``(B, T, Hq, D)`` (or written to ``q_out``).
    """
    return _lib.gpu_ops().rope_kv_write(q, k, v, cos, sin, k_dst, v_dst, k_scale_dst, v_scale_dst, block_table,
                                        start_pos, int(start_offset), int(page_size), bool(interleaved), q_out)


def quantize_kv_int8(x: torch.Tensor, scale_dtype: torch.dtype = torch.float16):
    """Per-(..., head_dim) symmetric int8 quantisation of a K or V tensor.

    x: (..., D) -> (int8 of the same shape, scale with the D axis dropped).
    ``scale = max|x| over D / 127`` (amax clamped to >= 1e-8 in x's dtype),
    ``xi = round(x / scale)`` half to even, clamped to +-127.  The scale is
    fp16 as in the reference (``model/kv_cache.py:67``); ``scale_dtype=float32``
    keeps it in fp32 (the paged pools' format).
    """
    ops = _lib.gpu_ops()
    if scale_dtype not in (torch.float16, torch.float32):
        raise ValueError("scale_dtype must be float16 or float32")
    src = x if x.stride(-1) == 1 and all((s * x.element_size()) % 16 == 0 for s in x.stride()[:-1]) \
        and x.data_ptr() % 16 == 0 else x.contiguous()
    return ops.quantize_kv_int8(src, scale_dtype == torch.float32)


def _int32_positions(pos: torch.Tensor) -> torch.Tensor:
    """Device positions as int32 (the reference's ctx.pos_index is int64)."""
    if pos.dtype == torch.int32:
        return pos
    if pos.dtype == torch.int64:
        return pos.to(torch.int32)
    raise ValueError("positions must be an int32 or int64 device tensor")


class KVCache:
    """Pre-allocated contiguous K/V pools for every layer (``model/kv_cache.py:70``)."""

    # Caches sized longer than this hold int8 K/V with fp16 scales (model/kv_cache.py:74,115)
    INT8_SEQ_THRESHOLD = 256

    def __init__(self, n_layers: int, max_batch: int, max_seq_len: int, n_heads_kv: int, head_dim: int,
                 dtype: torch.dtype = torch.bfloat16, device: torch.device | str = "cuda"):
        self.n_layers = n_layers
        self.max_batch = max_batch
        self.max_seq_len = max_seq_len
        self.n_heads_kv = n_heads_kv
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = torch.device(device)
        self.is_int8 = max_seq_len > KVCache.INT8_SEQ_THRESHOLD
        shape = (n_layers, max_batch, n_heads_kv, max_seq_len, head_dim)
        if self.is_int8:
            self.k_cache = torch.zeros(shape, dtype=torch.int8, device=self.device)
            self.v_cache = torch.zeros(shape, dtype=torch.int8, device=self.device)
            sshape = (n_layers, max_batch, n_heads_kv, max_seq_len)
            self.k_scale = torch.zeros(sshape, dtype=torch.float16, device=self.device)
            self.v_scale = torch.zeros(sshape, dtype=torch.float16, device=self.device)
        else:
            self.k_cache = torch.zeros(shape, dtype=dtype, device=self.device)
            self.v_cache = torch.zeros(shape, dtype=dtype, device=self.device)
            self.k_scale = self.v_scale = None

    def _layer(self, layer_idx: int, B: int):
        kc = self.k_cache[layer_idx, :B]
        vc = self.v_cache[layer_idx, :B]
        ks = self.k_scale[layer_idx, :B] if self.is_int8 else None
        vs = self.v_scale[layer_idx, :B] if self.is_int8 else None
        return kc, vc, ks, vs

    def update(self, layer_idx: int, start_pos: int, k: torch.Tensor, v: torch.Tensor):
        """Write K/V ``(B, Hkv, T, D)`` at ``[start_pos, start_pos + T)``.

        Returns what ``model/kv_cache.py:133-184`` returns: the cached prefix
        views ``(B, Hkv, start_pos + T, D)`` for a 16-bit cache, and the new
        ``k, v`` themselves for an int8 cache (whose prefix is read by the int8
        decode kernels instead).
        """
        B, H, T, D = k.shape
        end = start_pos + T
        assert B <= self.max_batch, f"batch {B} > max_batch {self.max_batch}"
        assert H == self.n_heads_kv, f"n_heads_kv mismatch: got {H}, expected {self.n_heads_kv}"
        assert D == self.head_dim, f"head_dim mismatch: got {D}, expected {self.head_dim}"
        assert end <= self.max_seq_len, f"sequence overflow: start_pos+T={end} > max_seq_len={self.max_seq_len}"
        kc, vc, ks, vs = self._layer(layer_idx, B)
        kv_write(k, v, kc, vc, ks, vs, start_offset=start_pos)
        if self.is_int8:
            return k, v
        return self.k_cache[layer_idx, :B, :, :end, :], self.v_cache[layer_idx, :B, :, :end, :]

    def write_decode(self, layer_idx: int, pos_index: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """Graph-safe single-step write of K/V ``(B, Hkv, 1, D)`` at the device position ``pos_index``.

        ``pos_index``: (1,) shared or (B,) per-sequence position on the device
        (int32, or int64 like the reference's ``ctx.pos_index``).  Positions
        past ``max_seq_len`` are skipped on the device.
        """
        B = k.shape[0]
        kc, vc, ks, vs = self._layer(layer_idx, B)
        kv_write(k, v, kc, vc, ks, vs, start_pos=_int32_positions(pos_index))

    def write_decode_rope(self, layer_idx: int, pos_index: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                          v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                          interleaved: bool = False) -> torch.Tensor:
        """RoPE + write of one decode step in one launch; returns the rotated q ``(B, 1, Hq, D)``.

        ``q, k, v``: the projections ``(B, 1, H, D)`` before RoPE
        (``ops/attention.py:200-202``); ``cos``/``sin``: the full tables
        (``RopeFrequencies.get(max_seq_len, dtype=...)``), read at each
        sequence's position ``pos_index`` on the device, so no per-step table
        row copy is needed.
        """
        B = k.shape[0]
        kc, vc, ks, vs = self._layer(layer_idx, B)
        return rope_kv_write(q, k, v, cos, sin, kc, vc, ks, vs, start_pos=_int32_positions(pos_index),
                             interleaved=interleaved)

    def reset(self) -> None:
        """Logical reset between independent sequences (nothing to clear, as in the reference)."""
        return

    def bytes(self) -> int:
        """Total footprint of the K and V pools in bytes."""
        return 2 * self.k_cache.numel() * self.k_cache.element_size()

    def __repr__(self) -> str:
        gb = self.bytes() / 1e9
        return (f"KVCache(n_layers={self.n_layers}, max_batch={self.max_batch}, max_seq_len={self.max_seq_len}, "
                f"n_heads_kv={self.n_heads_kv}, head_dim={self.head_dim}, dtype={self.dtype}, vram={gb:.2f} GB)")
