"""Decode attention (Tq == 1) entry points with the reference's signatures.

Each function is a drop-in for the reference function of the same name and
keeps its argument meaning, output layout and assertion behaviour; the work is
done by the gfx950 HIP kernels behind ``include/sia_attention.h``:

=================================  =================================================
this module                        reference
=================================  =================================================
attention_flash_decode             kernels/flash_decode_kernel.py:119-160
attention_flash_decode_int8        kernels/flash_decode_int8_kernel.py:121-167
paged_attention_flash_decode       kernels/paged_flash_decode_kernel.py:107-152
gqa_int8_flash_decode              kernels/paged_flash_decode_int8_gqa_kernel.py:100-124
paged_gqa_int8_flash_decode        (new: paged pool + int8 + GQA, BASELINE configs 3/5)
=================================  =================================================

Differences that only widen the reference's contract:

* ``kv_len`` may also be a ``(B,)`` int32 tensor (one length per sequence);
  a ``(1,)`` or ``()`` tensor keeps the reference's shared length.
* Long contexts are split across work-groups (split-K) and merged by a
  second kernel; the split is chosen on the device from ``kv_len``, so one
  captured HIP graph stays valid for every length.  Callers can pin the split
  with :func:`decode_options` (tests use it; the default is automatic).
"""

from __future__ import annotations

import contextlib
import threading

import torch

from . import _lib

_HEAD_DIMS = (16, 32, 64, 128, 256)
_tls = threading.local()
_ws_cache: dict = {}
# decode_options blocks active in any thread (their options are thread-local;
# with none active a call skips the thread-local lookups)
_opts_users = 0
_opts_lock = threading.Lock()
_OPS = None   # the extension module, once loaded on a GPU

# The reference wrappers assert; these raise the same AssertionError (even
# under -O), testing the condition first so that no message is formatted on
# a call that passes.


@contextlib.contextmanager
def decode_options(tiles_per_split: int = 0, main_events=None):
    """Options for decode calls made in this block (this thread).

    tiles_per_split: force the split-K size in 16-token tiles (0 = automatic).
    main_events: optional ``(begin, end)`` pair of timing ``torch.cuda.Event``
        (already recorded once, so that their HIP events exist); the library
        stamps them with the main decode kernel's own start and end
        (hipExtLaunchKernel; the split-K reduction is outside), for kernel
        timing.
    """
    global _opts_users
    prev = (getattr(_tls, "tiles_per_split", 0), getattr(_tls, "main_events", None))
    _tls.tiles_per_split = int(tiles_per_split)
    _tls.main_events = main_events
    with _opts_lock:
        _opts_users += 1
    try:
        yield
    finally:
        _tls.tiles_per_split, _tls.main_events = prev
        with _opts_lock:
            _opts_users -= 1


def decode_workspace_size(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int) -> int:
    """Bytes of split-K workspace a decode call of this geometry needs."""
    key = (batch, num_q_heads, num_kv_heads, head_dim, torch.cuda.current_device())
    n = _ws_cache.get(key)
    if n is None:
        n = _ws_cache[key] = int(_lib.gpu_ops().decode_workspace_size(batch, num_q_heads, num_kv_heads, head_dim))
    return n


def _kv_len_tensor(kv_len, device: torch.device) -> torch.Tensor:
    if isinstance(kv_len, torch.Tensor):
        if kv_len.dtype != torch.int32:
            raise ValueError("kv_len must be an int32 tensor")
        return kv_len
    # a device fill (no host-to-device copy), so the call can still be captured in a graph
    return torch.full((1,), int(kv_len), dtype=torch.int32, device=device)


# decode kinds of the extension's decode op (one per C entry point)
CONTIG, CONTIG_INT8, GQA_INT8, PAGED, PAGED_INT8 = range(5)


def _run(kind: int, q: torch.Tensor, k, v, k_scale, v_scale, block_table, kv_len, page_size: int,
         sm_scale: float) -> torch.Tensor:
    """One decode call through the torch extension (device checks, output and workspace in C++)."""
    global _OPS
    ops = _OPS
    if ops is None:
        ops = _OPS = _lib.gpu_ops()
    tps = b = e = 0
    if _opts_users:
        tps = getattr(_tls, "tiles_per_split", 0)
        ev = getattr(_tls, "main_events", None)
        if ev is not None:
            b, e = ev[0].cuda_event, ev[1].cuda_event
    return ops.decode(kind, q, k, v, k_scale, v_scale, block_table, kv_len, page_size, sm_scale, tps, b, e)


def _common(q: torch.Tensor, k: torch.Tensor, sm_scale):
    B, Hq, Tq, D = q.shape
    if Tq != 1:
        raise AssertionError("decode kernel expects a single query position")
    if D not in _HEAD_DIMS:
        raise AssertionError(f"unsupported head_dim {D}")
    return (1.0 / (D ** 0.5)) if sm_scale is None else float(sm_scale)


def attention_flash_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_len,
                           sm_scale: float | None = None) -> torch.Tensor:
    """Decode attention over a contiguous fp16/bf16 cache.

    q: (B, Hq, 1, D); k, v: (B, Hkv, S, D) (views into the preallocated cache);
    kv_len: int32 device tensor, (1,)/() shared or (B,) per sequence.
    Returns (B, 1, Hq, D) token-major in q's dtype.
    """
    scale = _common(q, k, sm_scale)
    kl = _kv_len_tensor(kv_len, q.device)
    return _run(CONTIG, q, k, v, None, None, None, kl, 0, scale)


def attention_flash_decode_int8(q: torch.Tensor, k_int8: torch.Tensor, v_int8: torch.Tensor,
                                k_scale: torch.Tensor, v_scale: torch.Tensor, kv_len,
                                sm_scale: float | None = None) -> torch.Tensor:
    """Decode attention over an int8 cache with per-(b, kv-head, pos) scales.

    k_int8, v_int8: (B, Hkv, S, D) int8; k_scale, v_scale: (B, Hkv, S) fp32 or fp16.
    """
    scale = _common(q, k_int8, sm_scale)
    kl = _kv_len_tensor(kv_len, q.device)
    return _run(CONTIG_INT8, q, k_int8, v_int8, k_scale, v_scale, None, kl, 0, scale)


def gqa_int8_flash_decode(q, k_int8, v_int8, k_scale, v_scale, kv_len, sm_scale=None):
    """GQA-grouped int8 decode: q (B, Hq, 1, D); k/v_int8 (B, Hkv, S, D); scales (B, Hkv, S).

    Every decode kernel here already reads each KV head once for its whole
    query-head group, so this shares the int8 kernel.
    """
    scale = _common(q, k_int8, sm_scale)
    kl = _kv_len_tensor(kv_len, q.device)
    return _run(GQA_INT8, q, k_int8, v_int8, k_scale, v_scale, None, kl, 0, scale)


def paged_attention_flash_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                                 block_table: torch.Tensor, kv_len, page_size: int,
                                 sm_scale: float | None = None) -> torch.Tensor:
    """Decode attention over a paged fp16/bf16 pool.

    k_pool, v_pool: (num_blocks, Hkv, page_size, D); block_table: (B, max_blocks)
    int32 logical->physical page ids.
    """
    Tq, D = q.shape[2], q.shape[3]
    P = k_pool.shape[2]
    # the reference's asserts, in its order (kernels/paged_flash_decode_kernel.py:131-134)
    if Tq != 1:
        raise AssertionError("decode kernel expects a single query position")
    if P != page_size:
        raise AssertionError(f"k_pool page dim {P} != page_size {page_size}")
    if D not in _HEAD_DIMS:
        raise AssertionError(f"unsupported head_dim {D}")
    scale = (1.0 / (D ** 0.5)) if sm_scale is None else float(sm_scale)
    kl = _kv_len_tensor(kv_len, q.device)
    return _run(PAGED, q, k_pool, v_pool, None, None, block_table, kl, page_size, scale)


def paged_gqa_int8_flash_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                                k_scale_pool: torch.Tensor, v_scale_pool: torch.Tensor,
                                block_table: torch.Tensor, kv_len, page_size: int,
                                sm_scale: float | None = None) -> torch.Tensor:
    """Paged INT8-KV GQA decode.

    k_pool, v_pool: (num_blocks, Hkv, page_size, D) int8; k_scale_pool,
    v_scale_pool: (num_blocks, Hkv, page_size) fp32 or fp16; block_table
    (B, max_blocks) int32; kv_len (1,)/() or (B,) int32.
    """
    Tq, D = q.shape[2], q.shape[3]
    P = k_pool.shape[2]
    # the reference's asserts, in its order (kernels/paged_flash_decode_kernel.py:131-134)
    if Tq != 1:
        raise AssertionError("decode kernel expects a single query position")
    if P != page_size:
        raise AssertionError(f"k_pool page dim {P} != page_size {page_size}")
    if D not in _HEAD_DIMS:
        raise AssertionError(f"unsupported head_dim {D}")
    scale = (1.0 / (D ** 0.5)) if sm_scale is None else float(sm_scale)
    kl = _kv_len_tensor(kv_len, q.device)
    return _run(PAGED_INT8, q, k_pool, v_pool, k_scale_pool, v_scale_pool, block_table, kl, page_size, scale)
