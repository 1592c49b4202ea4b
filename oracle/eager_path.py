"""Torch restatement of the reference's CPU/eager attention path.

TEST INFRASTRUCTURE ONLY -- used as a library-backed cross-check in ``tests/``
and as the timed CPU baseline (``cpu_baseline``, kind "port") in ``bench.py``.

The reference's eager path (``ops/attention.py:333-345``) repeats each KV head
``G = Hq // Hkv`` times with ``repeat_interleave`` and calls
``F.scaled_dot_product_attention(q, k, v, is_causal=T > 1)``, then transposes to
token-major ``(B, T, Hq, D)``.  Paged and int8 caches are first gathered by
block table and dequantised (``workspace/scripts/bench_paged_flash_jun28.py:17-38``,
``workspace/scripts/faith_int4_kv.py:10-15``), then go through the same code.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def eager_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool) -> torch.Tensor:
    """``ops/attention.py:333-345``: repeat_interleave GQA + SDPA, token-major out.

    q: (B, Hq, T, D); k, v: (B, Hkv, S, D).  Returns (B, T, Hq, D).
    """
    G = q.shape[1] // k.shape[1]
    if G > 1:
        k = k.repeat_interleave(G, dim=1)
        v = v.repeat_interleave(G, dim=1)
    out = F.scaled_dot_product_attention(q, k, v, attn_mask=None, dropout_p=0.0, is_causal=causal)
    return out.transpose(1, 2).contiguous()


def gather_pages(pool: torch.Tensor, block_table: torch.Tensor, b: int, n: int, page: int) -> torch.Tensor:
    """Pages of sequence b -> (Hkv, n, ...) (``workspace/scripts/bench_paged_flash_jun28.py:17-32``)."""
    t = torch.arange(n)
    phys = block_table[b, t // page].long()
    return pool[phys, :, t % page].movedim(0, 1)


def eager_paged_int8_decode(q, k_pool, v_pool, ks_pool, vs_pool, block_table, kv_len, page: int,
                            batch_rows=None) -> torch.Tensor:
    """Reference CPU path for paged INT8-KV decode: gather, dequantise, eager GQA.

    q: (B, Hq, 1, D) float32 on CPU.  ``batch_rows`` limits the work to a subset
    of sequences (the bounded CPU-baseline sample).  Returns (len(rows), 1, Hq, D).
    """
    rows = range(q.shape[0]) if batch_rows is None else batch_rows
    outs = []
    for b in rows:
        n = int(kv_len[b])
        k = gather_pages(k_pool, block_table, b, n, page).float() * \
            gather_pages(ks_pool, block_table, b, n, page).float()[..., None]
        v = gather_pages(v_pool, block_table, b, n, page).float() * \
            gather_pages(vs_pool, block_table, b, n, page).float()[..., None]
        outs.append(eager_gqa(q[b:b + 1], k[None], v[None], causal=False))
    return torch.cat(outs, 0)

