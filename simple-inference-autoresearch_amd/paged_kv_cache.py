"""Block-paged K/V cache with the reference's interface, written on the GPU.

Drop-in for ``model/paged_kv_cache.py`` (``PagedKVCache``, lines 38-115):
same constructor, pools ``(L, num_blocks, Hkv, block_size, D)``,
``block_tables (max_batch, max_blocks_per_seq) int32``, ``seq_lens
(max_batch,) int32``, bump ``allocate`` and ``write_prefill``.  Differences,
all widening the contract:

* ``write_prefill`` is one HIP launch (``sia_kv_write``) instead of a Python
  loop of slice copies, and writes where the reference's loop writes (token
  ``t`` of request ``b`` to block ``b * max_blocks_per_seq + t // block_size``).
* ``kv_dtype=torch.int8`` stores int8 pools with fp32 per-token-per-head scale
  pools ``(L, num_blocks, Hkv, block_size)`` (the format of the paged INT8-KV
  GQA decode kernel); writes quantise on the fly.
* The decode-step write that the reference documents but never implements
  (``slot_for``, ``model/paged_kv_cache.py:29-30``) is :meth:`write_decode`:
  the slot is derived on the device from ``seq_lens`` through the block table,
  so one captured HIP graph serves every step.  ``seq_lens`` counts the tokens
  stored per request including the one being decoded: :meth:`begin_decode_step`
  bumps it once per step, :meth:`write_decode` writes at ``seq_lens[b] - 1``
  and :meth:`decode_attention` attends over ``seq_lens[b]`` tokens.
"""

from __future__ import annotations

import torch

from .decode import paged_attention_flash_decode, paged_gqa_int8_flash_decode
from .kv_cache import kv_write, rope_kv_write


class PagedKVCache:
    BACKEND = "paged"

    def __init__(self, n_layers, max_batch, max_seq_len, n_heads_kv, head_dim, block_size=16,
                 dtype=torch.bfloat16, device="cuda", kv_dtype: torch.dtype | None = None):
        self.n_layers = n_layers
        self.max_batch = max_batch
        self.max_seq_len = max_seq_len
        self.n_heads_kv = n_heads_kv
        self.head_dim = head_dim
        self.block_size = block_size
        self.dtype = dtype
        self.device = torch.device(device)
        self.kv_dtype = dtype if kv_dtype is None else kv_dtype
        if self.kv_dtype not in (torch.float16, torch.bfloat16, torch.int8):
            raise ValueError("kv_dtype must be float16, bfloat16 or int8")
        self.is_int8 = self.kv_dtype == torch.int8

        self.max_blocks_per_seq = (max_seq_len + block_size - 1) // block_size
        # one full max_seq_len per request, as the reference sizes it
        self.num_blocks = max_batch * self.max_blocks_per_seq
        shape = (n_layers, self.num_blocks, n_heads_kv, block_size, head_dim)
        self.k_pool = torch.zeros(shape, dtype=self.kv_dtype, device=self.device)
        self.v_pool = torch.zeros(shape, dtype=self.kv_dtype, device=self.device)
        if self.is_int8:
            sshape = (n_layers, self.num_blocks, n_heads_kv, block_size)
            self.k_scale_pool = torch.zeros(sshape, dtype=torch.float32, device=self.device)
            self.v_scale_pool = torch.zeros(sshape, dtype=torch.float32, device=self.device)
        else:
            self.k_scale_pool = self.v_scale_pool = None

        self.block_tables = torch.zeros(max_batch, self.max_blocks_per_seq, dtype=torch.int32, device=self.device)
        self.seq_lens = torch.zeros(max_batch, dtype=torch.int32, device=self.device)
        # request b's sequential block ids: where write_prefill puts the prompt
        # (model/paged_kv_cache.py:93-109 writes to b * max_blocks_per_seq + t // bs)
        self._prefill_table = (torch.arange(max_batch, dtype=torch.int32, device=self.device)[:, None]
                               * self.max_blocks_per_seq
                               + torch.arange(self.max_blocks_per_seq, dtype=torch.int32, device=self.device)[None])
        self._next_free = 0
        self._allocated_B = 0

    # -- allocation (model/paged_kv_cache.py:67-86) -----------------------------------
    def reset(self) -> None:
        self._next_free = 0
        self._allocated_B = 0
        self.seq_lens.zero_()

    def allocate(self, B: int, n_blocks_per_seq: int) -> None:
        """Give each of the B requests ``n_blocks_per_seq`` sequential physical blocks."""
        assert B <= self.max_batch
        assert n_blocks_per_seq <= self.max_blocks_per_seq
        self.block_tables[:B, :n_blocks_per_seq].copy_(self._prefill_table[:B, :n_blocks_per_seq])
        self._allocated_B = B
        self._next_free = B * self.max_blocks_per_seq

    # -- views ----------------------------------------------------------------------
    def layer(self, layer_idx: int):
        """(k_pool, v_pool, k_scale_pool, v_scale_pool) of one layer (scales None unless int8)."""
        ks = self.k_scale_pool[layer_idx] if self.is_int8 else None
        vs = self.v_scale_pool[layer_idx] if self.is_int8 else None
        return self.k_pool[layer_idx], self.v_pool[layer_idx], ks, vs

    # -- writes ---------------------------------------------------------------------
    def write_prefill(self, layer_idx: int, B: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Scatter the prompt K/V ``(B, Hkv, T, D)`` into the pool (one launch)."""
        T = k.shape[2]
        assert T <= self.max_blocks_per_seq * self.block_size, "prompt longer than max_seq_len"
        kp, vp, ks, vs = self.layer(layer_idx)
        kv_write(k[:B], v[:B], kp, vp, ks, vs, block_table=self._prefill_table[:B], page_size=self.block_size)

    def set_lengths(self, B: int, n: int) -> None:
        """Record that requests ``[0, B)`` hold ``n`` tokens (e.g. the prompt length after prefill)."""
        self.seq_lens[:B].fill_(n)

    def begin_decode_step(self, B: int) -> None:
        """Count the token this decode step adds (``seq_lens[:B] += 1``, on the device)."""
        self.seq_lens[:B].add_(1)

    def write_decode(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write this step's K/V ``(B, Hkv, 1, D)`` at position ``seq_lens[b] - 1`` via the block table."""
        B = k.shape[0]
        kp, vp, ks, vs = self.layer(layer_idx)
        kv_write(k, v, kp, vp, ks, vs, block_table=self.block_tables[:B], start_pos=self.seq_lens[:B],
                 start_offset=-1, page_size=self.block_size)

    def write_decode_rope(self, layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          cos: torch.Tensor, sin: torch.Tensor, interleaved: bool = False) -> torch.Tensor:
        """RoPE + paged write of this step's token in one launch; returns the rotated q ``(B, 1, Hq, D)``.

        ``q, k, v``: projections ``(B, 1, H, D)`` before RoPE.  Request ``b``'s
        token sits at position ``seq_lens[b] - 1`` (read on the device) and is
        rotated by that row of the full ``cos``/``sin`` tables, so requests at
        different positions share one launch.
        """
        B = k.shape[0]
        kp, vp, ks, vs = self.layer(layer_idx)
        return rope_kv_write(q, k, v, cos, sin, kp, vp, ks, vs, block_table=self.block_tables[:B],
                             start_pos=self.seq_lens[:B], start_offset=-1, page_size=self.block_size,
                             interleaved=interleaved)

    def decode_attention(self, layer_idx: int, q: torch.Tensor, sm_scale: float | None = None) -> torch.Tensor:
        """Decode attention of ``q (B, Hq, 1, D)`` over each request's ``seq_lens[b]`` cached tokens."""
        B = q.shape[0]
        kp, vp, ks, vs = self.layer(layer_idx)
        if self.is_int8:
            return paged_gqa_int8_flash_decode(q, kp, vp, ks, vs, self.block_tables[:B], self.seq_lens[:B],
                                               self.block_size, sm_scale)
        return paged_attention_flash_decode(q, kp, vp, self.block_tables[:B], self.seq_lens[:B],
                                            self.block_size, sm_scale)

    def __repr__(self):
        gb = 2 * self.k_pool.numel() * self.k_pool.element_size() / 1e9
        return (f"PagedKVCache(layers={self.n_layers}, blocks={self.num_blocks}, block_size={self.block_size}, "
                f"max_batch={self.max_batch}, max_seq_len={self.max_seq_len}, kv_dtype={self.kv_dtype}, "
                f"vram={gb:.2f} GB)")
