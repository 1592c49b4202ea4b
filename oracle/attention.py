"""Float64 numpy restatement of the reference attention path (test oracle).

TEST INFRASTRUCTURE ONLY -- imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``; never by the product package.

Every function cites the reference lines whose behaviour it restates
(paths relative to the reference repository root).  All arithmetic that the
reference does in floating point is done here in float64, so the oracle is a
tighter reference than any fp32/bf16 implementation; the one exception is
``quantize_kv_int8``, whose *integer* output is defined by float32 arithmetic
in the reference and is therefore reproduced in float32, bit for bit.
"""

from __future__ import annotations

import math

import numpy as np

# ---------------------------------------------------------------------------
# dtype helpers (numpy has no bfloat16; bf16 values are carried in float32)
# ---------------------------------------------------------------------------


def round_to_bf16(x) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), as float32."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    bits = a.view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    rounded = ((bits + 0x7FFF + lsb) >> 16) << 16
    out = (rounded & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    # NaN stays NaN (the rounding above could otherwise turn a NaN into inf)
    return np.where(np.isnan(a), a, out)


def round_to_dtype(x, dtype: str) -> np.ndarray:
    """Round values to ``dtype`` ('float32' | 'float16' | 'bfloat16'), as float32."""
    if dtype == "float32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "float16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return round_to_bf16(x)
    raise ValueError(f"unsupported dtype {dtype!r}")


# ---------------------------------------------------------------------------
# INT8 KV format
# ---------------------------------------------------------------------------


def quantize_kv_int8(x, src_dtype: str = "float32", scale_dtype: str = "float16"):
    """Per-vector symmetric int8 quantisation over the last axis.

    Restates ``model/kv_cache.py:58-67``::

        amax  = x.abs().amax(-1, keepdim=True).clamp_min(1e-8).float()
        scale = amax / 127.0
        xi    = round(x.float() / scale).clamp(-127, 127).to(int8)
        return xi, scale.squeeze(-1).to(float16)

    ``x`` holds values already representable in ``src_dtype`` (the tensor dtype
    the reference sees); the 1e-8 floor is applied in that dtype, exactly as
    ``clamp_min`` does on a tensor of that dtype.  ``scale_dtype`` is 'float16'
    for the reference ``KVCache`` and 'float32' for the per-token-per-head fp32
    scales of the paged pools (``workspace/scripts/bench_flash_int8_jun27.py:25-30``).
    Division and rounding are float32 and round-half-to-even, as in torch.
    """
    x32 = np.asarray(x, dtype=np.float32)
    floor = np.float32(round_to_dtype(np.float32(1e-8), src_dtype))
    amax = np.max(np.abs(x32), axis=-1, keepdims=True).astype(np.float32)
    amax = np.maximum(amax, floor)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    # an all-zero fp16 row has scale 0 (1e-8 rounds to 0 in fp16): 0 / 0 is
    # NaN, which torch's float -> int8 conversion turns into 0; stated
    # explicitly here (numpy's NaN -> int8 cast is platform-defined)
    with np.errstate(invalid="ignore", divide="ignore"):
        xi = np.rint((x32 / scale).astype(np.float32))
    xi = np.where(np.isnan(xi), np.float32(0.0), xi)
    xi = np.clip(xi, -127, 127).astype(np.int8)
    scale = np.squeeze(scale, -1)
    if scale_dtype == "float16":
        scale = scale.astype(np.float16)
    elif scale_dtype != "float32":
        raise ValueError(f"unsupported scale dtype {scale_dtype!r}")
    return xi, scale


def dequantize_int8(xi, scale) -> np.ndarray:
    """``xi * scale[..., None]`` in float64: the reference's dequantised values.

    The int8 kernels fold the scales into the math (``qk *= s_k`` after the dot,
    ``p *= s_v`` before PV: ``kernels/flash_decode_int8_kernel.py:98,111-112``),
    which is exactly attention over these dequantised K/V.
    """
    return np.asarray(xi, dtype=np.float64) * np.asarray(scale, dtype=np.float64)[..., None]


# ---------------------------------------------------------------------------
# decode (Tq == 1)
# ---------------------------------------------------------------------------


def _kv_lens(kv_len, B: int) -> np.ndarray:
    """Broadcast a scalar / (1,) / (B,) kv_len to one length per sequence."""
    a = np.asarray(kv_len, dtype=np.int64).reshape(-1)
    if a.size == 1:
        return np.full(B, int(a[0]), dtype=np.int64)
    if a.size != B:
        raise ValueError(f"kv_len has {a.size} entries, expected 1 or {B}")
    return a


def _decode_one(q_b, k_b, v_b, n: int, scale: float) -> np.ndarray:
    """One sequence: q_b (Hq, D), k_b/v_b (Hkv, >=n, D) -> (Hq, D) float64.

    Query head hq reads KV head hq // (Hq // Hkv)
    (``kernels/flash_decode_kernel.py:70-73``).  An empty prefix gives zeros,
    the reference's ``l_safe`` guard (``kernels/flash_decode_kernel.py:113-114``).
    """
    Hq, D = q_b.shape
    Hkv = k_b.shape[0]
    G = Hq // Hkv
    out = np.zeros((Hq, D), dtype=np.float64)
    if n <= 0:
        return out
    for h in range(Hkv):
        qg = np.asarray(q_b[h * G:(h + 1) * G], dtype=np.float64)      # (G, D)
        kh = np.asarray(k_b[h, :n], dtype=np.float64)                   # (n, D)
        vh = np.asarray(v_b[h, :n], dtype=np.float64)
        s = (qg @ kh.T) * scale                                         # (G, n)
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        out[h * G:(h + 1) * G] = (p @ vh) / p.sum(axis=1, keepdims=True)
    return out


def gqa_decode(q, k, v, kv_len, sm_scale: float | None = None) -> np.ndarray:
    """Single-query GQA decode over a contiguous cache.

    Restates ``attention_flash_decode`` (``kernels/flash_decode_kernel.py:53-160``)
    and the eager path it replaces (``ops/attention.py:333-345``): for each
    sequence b and query head hq, ``softmax(q k^T * scale) v`` over keys
    ``[0, kv_len_b)`` of KV head ``hq // G``.

    q: (B, Hq, 1, D); k, v: (B, Hkv, S, D); kv_len: int, (1,) or (B,).
    Returns (B, 1, Hq, D) float64 (token-major, like the reference).
    """
    q = np.asarray(q)
    B, Hq, Tq, D = q.shape
    if Tq != 1:
        raise ValueError("decode expects a single query position")
    S = k.shape[2]
    lens = _kv_lens(kv_len, B)
    if (lens > S).any() or (lens < 0).any():
        raise ValueError("kv_len outside [0, S]")
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    out = np.zeros((B, 1, Hq, D), dtype=np.float64)
    for b in range(B):
        out[b, 0] = _decode_one(q[b, :, 0], k[b], v[b], int(lens[b]), scale)
    return out


def int8_decode(q, k_int8, v_int8, k_scale, v_scale, kv_len, sm_scale=None) -> np.ndarray:
    """INT8-KV decode: ``gqa_decode`` over the dequantised cache.

    Restates ``attention_flash_decode_int8`` (``kernels/flash_decode_int8_kernel.py:51-167``)
    and ``gqa_int8_flash_decode`` (``kernels/paged_flash_decode_int8_gqa_kernel.py:31-124``):
    both compute attention over ``k_int8*s_k``, ``v_int8*s_v``.
    k_int8/v_int8: (B, Hkv, S, D); k_scale/v_scale: (B, Hkv, S).
    """
    return gqa_decode(q, dequantize_int8(k_int8, k_scale), dequantize_int8(v_int8, v_scale),
                      kv_len, sm_scale)


# ---------------------------------------------------------------------------
# paged layout
# ---------------------------------------------------------------------------


def paged_gather(pool, block_table, b: int, n_tokens: int, page_size: int) -> np.ndarray:
    """Gather tokens [0, n_tokens) of sequence b from a paged pool.

    Token t of sequence b lives at ``pool[block_table[b, t // page], :, t % page]``
    (``kernels/paged_flash_decode_kernel.py:74-84``;
    pool layout ``(num_blocks, Hkv, page, ...)``, ``model/paged_kv_cache.py:18-24``).
    Returns (Hkv, n_tokens, ...) in the pool's dtype.
    """
    pool = np.asarray(pool)
    bt = np.asarray(block_table)
    t = np.arange(n_tokens)
    phys = bt[b, t // page_size]
    g = pool[phys, :, t % page_size]            # (n, Hkv, ...)
    return np.moveaxis(g, 0, 1)


def paged_decode(q, k_pool, v_pool, block_table, kv_len, page_size: int, sm_scale=None) -> np.ndarray:
    """Paged fp16/bf16 decode: gather by block table, then ``gqa_decode``.

    Restates ``paged_attention_flash_decode`` (``kernels/paged_flash_decode_kernel.py:40-152``),
    with ``kv_len`` widened to one length per sequence.
    """
    q = np.asarray(q)
    B, Hq, _, D = q.shape
    lens = _kv_lens(kv_len, B)
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    out = np.zeros((B, 1, Hq, D), dtype=np.float64)
    for b in range(B):
        n = int(lens[b])
        k_b = paged_gather(k_pool, block_table, b, n, page_size)
        v_b = paged_gather(v_pool, block_table, b, n, page_size)
        out[b, 0] = _decode_one(q[b, :, 0], k_b, v_b, n, scale)
    return out


def paged_int8_decode(q, k_pool, v_pool, k_scale_pool, v_scale_pool, block_table, kv_len,
                      page_size: int, sm_scale=None) -> np.ndarray:
    """Paged INT8-KV GQA decode (BASELINE config 3/5 composition).

    Gathers int8 pages ``(NB, Hkv, page, D)`` and their scales ``(NB, Hkv, page)``
    by block table (``kernels/paged_flash_decode_kernel.py:74-84``), dequantises
    (``kernels/flash_decode_int8_kernel.py:98,111-112``) and attends
    (``kernels/paged_flash_decode_int8_gqa_kernel.py:47-97``).
    """
    q = np.asarray(q)
    B, Hq, _, D = q.shape
    lens = _kv_lens(kv_len, B)
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    out = np.zeros((B, 1, Hq, D), dtype=np.float64)
    for b in range(B):
        n = int(lens[b])
        k_b = dequantize_int8(paged_gather(k_pool, block_table, b, n, page_size),
                              paged_gather(k_scale_pool, block_table, b, n, page_size))
        v_b = dequantize_int8(paged_gather(v_pool, block_table, b, n, page_size),
                              paged_gather(v_scale_pool, block_table, b, n, page_size))
        out[b, 0] = _decode_one(q[b, :, 0], k_b, v_b, n, scale)
    return out


# ---------------------------------------------------------------------------
# split-K (FlashDecoding) partials and merge
# ---------------------------------------------------------------------------


def decode_partial(q_g, k_h, v_h, lo: int, hi: int, scale: float):
    """Partial softmax state of query rows q_g (G, D) over keys [lo, hi).

    Returns (m, l, acc): m (G,) running max (-inf when empty), l (G,) = sum
    exp(s - m), acc (G, D) = sum exp(s - m) v.  The same (m, l, acc) recurrence
    as the reference's online softmax (``kernels/attention_kernel.py:211-222``).
    """
    G, D = q_g.shape
    if hi <= lo:
        return np.full(G, -np.inf), np.zeros(G), np.zeros((G, D))
    s = (np.asarray(q_g, np.float64) @ np.asarray(k_h[lo:hi], np.float64).T) * scale
    m = s.max(axis=1)
    p = np.exp(s - m[:, None])
    return m, p.sum(axis=1), p @ np.asarray(v_h[lo:hi], np.float64)


def merge_partials(parts) -> np.ndarray:
    """Merge split-K partials: M = max m_i, L = sum l_i e^(m_i-M), O = sum acc_i e^(m_i-M) / L.

    Empty partials (m = -inf) contribute nothing; if every partial is empty the
    result is zero, matching the reference's ``l_safe`` guard.
    """
    ms = np.stack([p[0] for p in parts])                     # (n, G)
    M = ms.max(axis=0)
    Msafe = np.where(np.isfinite(M), M, 0.0)
    w = np.where(np.isfinite(ms), np.exp(ms - Msafe), 0.0)    # (n, G)
    L = sum(w[i] * parts[i][1] for i in range(len(parts)))
    A = sum(w[i][:, None] * parts[i][2] for i in range(len(parts)))
    Lsafe = np.where(L == 0.0, 1.0, L)
    return A / Lsafe[:, None]


# ---------------------------------------------------------------------------
# prefill / general attention (any Tq), causal with bottom-right offset
# ---------------------------------------------------------------------------


def flash_attention(q, k, v, causal: bool, sm_scale: float | None = None) -> np.ndarray:
    """General GQA attention, any Tq, optional causal mask with a Tk-Tq offset.

    Restates ``_flash_fwd`` / ``attention_flash_triton``
    (``kernels/attention_kernel.py:165-232,235-305``): query row i sits at
    absolute position ``(Tk - Tq) + i`` and, when causal, attends to keys
    ``j <= (Tk - Tq) + i``; a fully masked row is written as zeros (224-226);
    GQA maps query head hq to KV head ``hq // (Hq // Hkv)`` (169).

    q: (B, Hq, Tq, D); k, v: (B, Hkv, Tk, D).  Returns (B, Hq, Tq, D) float64.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, Tq, D = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    out = np.zeros((B, Hq, Tq, D), dtype=np.float64)
    if causal:
        allowed = np.arange(Tk)[None, :] <= (Tk - Tq) + np.arange(Tq)[:, None]   # (Tq, Tk)
    else:
        allowed = np.ones((Tq, Tk), dtype=bool)
    live = allowed.any(axis=1)                                                 # (Tq,)
    for b in range(B):
        for hq in range(Hq):
            h = hq // G
            s = (q[b, hq] @ k[b, h].T) * scale                                 # (Tq, Tk)
            s = np.where(allowed, s, -np.inf)
            m = np.where(live, s.max(axis=1), 0.0)
            p = np.where(allowed, np.exp(s - m[:, None]), 0.0)
            l = p.sum(axis=1)
            o = (p @ v[b, h]) / np.where(l == 0.0, 1.0, l)[:, None]
            out[b, hq] = o
    return out


# ---------------------------------------------------------------------------
# KV write path
# ---------------------------------------------------------------------------


def kv_write_positions(B: int, T: int, start, start_offset: int = 0) -> np.ndarray:
    """Position of token t of sequence b: ``start_offset + start[b] + t`` -> (B, T) int64.

    ``start`` is a scalar or one value per sequence; the reference's writes use
    ``start_pos`` (``model/kv_cache.py:146,178-179``) and, in the captured
    decode step, the device position ``ctx.pos_index`` (``ops/attention.py:221-228``).
    """
    s = np.asarray(start, dtype=np.int64).reshape(-1)
    s = np.full(B, int(s[0])) if s.size == 1 else s
    return start_offset + s[:, None] + np.arange(T)[None, :]


def kv_write_contiguous(cache, x, start, start_offset: int = 0):
    """Store x (B, H, T, ...) into cache (B', H, S, ...) at the positions above; positions
    outside [0, S) are dropped.  Restates the slice assignment of
    ``model/kv_cache.py:167-180``.  Returns a new array."""
    out = np.array(cache, copy=True)
    B, H, T = x.shape[:3]
    pos = kv_write_positions(B, T, start, start_offset)
    for b in range(B):
        for t in range(T):
            p = int(pos[b, t])
            if 0 <= p < out.shape[2]:
                out[b, :, p] = x[b, :, t]
    return out


def kv_write_paged(pool, x, block_table, page_size: int, start, start_offset: int = 0):
    """Store x (B, H, T, ...) into pool (num_pages, H, page_size, ...): position p of
    sequence b goes to page ``block_table[b][p // page_size]``, offset ``p % page_size``
    (``model/paged_kv_cache.py:89-109``); positions past the table or pages outside
    the pool are dropped.  Returns a new array."""
    out = np.array(pool, copy=True)
    bt = np.asarray(block_table)
    B, H, T = x.shape[:3]
    pos = kv_write_positions(B, T, start, start_offset)
    for b in range(B):
        for t in range(T):
            p = int(pos[b, t])
            if p < 0 or p // page_size >= bt.shape[1]:
                continue
            pg = int(bt[b, p // page_size])
            if 0 <= pg < out.shape[0]:
                out[pg, :, p % page_size] = x[b, :, t]
    return out
