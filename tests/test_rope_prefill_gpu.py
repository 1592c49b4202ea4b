"""GPU parity of the prefill kernel with q rotated at load (``rope_attention_flash_triton``).

Two bars:
  * bit-exact against the unfused pair it replaces on the GPU -- ``rope_triton``
    on q (``kernels/rope_kernel.py:261``) then ``attention_flash_triton``
    (``ops/attention.py:291-292, 327-330``): the fused prologue rotates with the
    same fp32 arithmetic and rounding, so the MFMA kernel sees the same q bits;
  * against the float64 oracle composed from pinned pieces -- ``oracle.rope.rope_qk``
    (pinned to transformers' rotary functions) then ``oracle.attention.flash_attention``
    (pinned to SDPA and brute-force golden vectors) -- with the prefill tests'
    tolerance: max-abs <= 2e-3 before one rounding to the output dtype.
A query whose position has no table row (device-read positions only) is
rotated to zeros, so its attention weights are uniform: its output is the mean
of the visible V rows, a closed form checked here.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import announce, assert_close, f64
from oracle import attention as O
from oracle import rope as OR

pytestmark = pytest.mark.gpu
DEV = "cuda"
_NP_DT = {torch.bfloat16: "bfloat16", torch.float16: "float16"}


def check(out, ref, what, atol=2e-3):
    assert_close(out, ref, atol, what)


def tables(Tc, D, dtype, half_width=False, theta=10000.0):
    inv = 1.0 / theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = torch.outer(torch.arange(Tc, dtype=torch.float64), inv)
    c, s = ang.cos(), ang.sin()
    if not half_width:
        c, s = torch.cat([c, c], -1), torch.cat([s, s], -1)
    return c.to(dtype).to(DEV), s.to(dtype).to(DEV)


def inputs(B, Hq, Hkv, Tq, Tk, D, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = (torch.randn(B, Hq, Tq, D, generator=g, device=DEV) * 0.5).to(dtype)
    k = (torch.randn(B, Hkv, Tk, D, generator=g, device=DEV) * 0.5).to(dtype)
    v = (torch.randn(B, Hkv, Tk, D, generator=g, device=DEV) * 0.5).to(dtype)
    return q, k, v


def unfused(pkg, q, k, v, cos, sin, starts, interleaved, causal):
    """rope_triton on q (table rows starts[b] + i) then attention_flash_triton, per sequence."""
    outs = []
    Tq = q.shape[2]
    for b, s0 in enumerate(starts):
        qb = q[b:b + 1].transpose(1, 2)                         # (1, Tq, Hq, D) view
        qr, _ = pkg.rope_triton(qb, qb[:, :, :1], cos[s0:s0 + Tq], sin[s0:s0 + Tq], interleaved=interleaved)
        outs.append(pkg.attention_flash_triton(qr.transpose(1, 2), k[b:b + 1], v[b:b + 1], causal=causal))
    return torch.cat(outs, 0)


def oracle(q, k, v, cos, sin, starts, interleaved, causal):
    """float64 oracle: oracle rope of q at rows starts[b] + i, rounded to q's dtype, then flash attention."""
    dt = _NP_DT[q.dtype]
    Tq = q.shape[2]
    qn = np.transpose(f64(q), (0, 2, 1, 3))                       # (B, Tq, Hq, D)
    rot = np.empty_like(qn)
    for b, s0 in enumerate(starts):
        c, s = f64(cos)[s0:s0 + Tq], f64(sin)[s0:s0 + Tq]
        rot[b:b + 1], _ = OR.rope_qk(qn[b:b + 1], qn[b:b + 1, :, :1], c, s, interleaved=interleaved, dtype=dt)
    return O.flash_attention(np.transpose(rot, (0, 2, 1, 3)), f64(k), f64(v), causal)


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("interleaved", [False, True])
def test_fused_equals_rope_then_attention(gpu_pkg, D, dtype, interleaved):
    B, Hq, Hkv, T = 2, 8, 2, 130
    announce(f"rope prefill D={D} {dtype} il={interleaved}")
    q, k, v = inputs(B, Hq, Hkv, T, T, D, dtype, seed=D + (7 if interleaved else 0))
    cos, sin = tables(T + 40, D, torch.float32 if D == 64 else dtype, half_width=D == 128)
    got = gpu_pkg.rope_attention_flash_triton(q, k, v, cos, sin, causal=True, start_offset=9,
                                              interleaved=interleaved)
    want = unfused(gpu_pkg, q, k, v, cos, sin, [9] * B, interleaved, True)
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"fused differs from rope_triton + attention (max {(got - want).abs().max()})"
    check(got, oracle(q, k, v, cos, sin, [9] * B, interleaved, True), f"D={D} il={interleaved}")


@pytest.mark.parametrize("Tq,Tk,causal", [(64, 300, True), (200, 513, True), (512, 512, True), (17, 17, False),
                                          (300, 64, False)])
def test_chunked_and_full(gpu_pkg, Tq, Tk, causal):
    """Chunked prefill (Tq < Tk, queries at positions Tk - Tq + i) and non-causal attention."""
    announce(f"rope prefill Tq={Tq} Tk={Tk} causal={causal}")
    q, k, v = inputs(1, 16, 4, Tq, Tk, 128, torch.bfloat16, seed=Tq + Tk)
    cos, sin = tables(max(Tq, Tk) + 8, 128, torch.bfloat16)
    s0 = max(Tk - Tq, 0)
    got = gpu_pkg.rope_attention_flash_triton(q, k, v, cos, sin, causal=causal, start_offset=s0,
                                              out_token_major=True)
    want = unfused(gpu_pkg, q, k, v, cos, sin, [s0], False, causal)
    torch.cuda.synchronize()
    assert got.shape == (1, Tq, 16, 128)
    assert torch.equal(got.transpose(1, 2), want)
    check(got.transpose(1, 2), oracle(q, k, v, cos, sin, [s0], False, causal), f"Tq={Tq} Tk={Tk}")


def test_device_start_positions_per_sequence(gpu_pkg):
    """Positions read on the device: start_offset + start_pos[b] + i, one start per sequence."""
    B, Hq, Hkv, T, D = 3, 8, 2, 70, 128
    announce("rope prefill device start_pos per sequence")
    q, k, v = inputs(B, Hq, Hkv, T, T, D, torch.float16, seed=3)
    cos, sin = tables(256, D, torch.float16)
    sp = torch.tensor([0, 50, 120], dtype=torch.int32, device=DEV)
    got = gpu_pkg.rope_attention_flash_triton(q, k, v, cos, sin, causal=True, start_pos=sp, start_offset=4)
    starts = [4, 54, 124]
    want = unfused(gpu_pkg, q, k, v, cos, sin, starts, False, True)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    check(got, oracle(q, k, v, cos, sin, starts, False, True), "per-sequence starts")
    # one shared device start
    one = torch.tensor([33], dtype=torch.int32, device=DEV)
    got1 = gpu_pkg.rope_attention_flash_triton(q, k, v, cos, sin, causal=True, start_pos=one)
    torch.cuda.synchronize()
    assert torch.equal(got1, unfused(gpu_pkg, q, k, v, cos, sin, [33] * B, False, True))


def test_rows_without_table_row_attend_uniformly(gpu_pkg):
    """A device position past the table rotates q to zeros: uniform weights, output = mean of visible V."""
    B, Hq, Hkv, T, D = 1, 4, 1, 96, 64
    announce("rope prefill positions past the table")
    q, k, v = inputs(B, Hq, Hkv, T, T, D, torch.bfloat16, seed=11)
    Tc = 60
    cos, sin = tables(Tc, D, torch.bfloat16)
    sp = torch.tensor([20], dtype=torch.int32, device=DEV)      # rows i >= 40 sit past the table
    got = gpu_pkg.rope_attention_flash_triton(q, k, v, cos, sin, causal=True, start_pos=sp)
    torch.cuda.synchronize()
    inside = Tc - 20
    ref_in = oracle(q[:, :, :inside], k[:, :, :inside], v[:, :, :inside], cos, sin, [20], False, True)
    check(got[:, :, :inside], ref_in, "rows inside the table")
    vf = f64(v)[0, 0]
    mean = np.cumsum(vf, axis=0) / np.arange(1, T + 1)[:, None]    # row i sees keys 0..i
    check(got[0, :, inside:], np.broadcast_to(mean[inside:], (Hq, T - inside, D)), "rows past the table")


def test_kv_write_then_fused_prefill_pipeline(gpu_pkg):
    """rope_kv_write(q=None) fills the cache with rotated K; the fused prefill rotates q itself.

    Equals the reference order -- rope_triton(q, k), cache update, attention
    (``ops/attention.py:291-330``) -- bit for bit.
    """
    B, Hq, Hkv, T, D, S = 2, 8, 2, 100, 128, 160
    announce("rope_kv_write + fused rope prefill pipeline")
    g = torch.Generator(device=DEV).manual_seed(5)
    qkv = torch.randn(B, T, (Hq + 2 * Hkv) * D, generator=g, device=DEV).to(torch.bfloat16)
    q = qkv[..., :Hq * D].reshape(B, T, Hq, D)
    k = qkv[..., Hq * D:(Hq + Hkv) * D].reshape(B, T, Hkv, D)
    v = qkv[..., (Hq + Hkv) * D:].reshape(B, T, Hkv, D)
    cos, sin = tables(S, D, torch.bfloat16)
    kc = torch.zeros(B, Hkv, S, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    gpu_pkg.rope_kv_write(None, k, v, cos, sin, kc, vc)
    got = gpu_pkg.rope_attention_flash_triton(q.transpose(1, 2), kc[:, :, :T], vc[:, :, :T], cos, sin,
                                              causal=True, out_token_major=True)
    qr, kr = gpu_pkg.rope_triton(q, k, cos[:T], sin[:T])
    want = gpu_pkg.attention_flash_triton(qr.transpose(1, 2), kr.transpose(1, 2), v.transpose(1, 2), causal=True,
                                          out_token_major=True)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_tables_in_another_16_bit_dtype(gpu_pkg):
    """bf16 q with f16 tables: the wrapper widens the tables to fp32 (exact), the result is unchanged."""
    B, Hq, Hkv, T, D = 1, 8, 2, 90, 128
    announce("rope prefill bf16 q, f16 tables")
    q, k, v = inputs(B, Hq, Hkv, T, T, D, torch.bfloat16, seed=21)
    cos, sin = tables(T, D, torch.float16)
    got = gpu_pkg.rope_attention_flash_triton(q, k, v, cos, sin, causal=True)
    want = unfused(gpu_pkg, q, k, v, cos, sin, [0], False, True)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    from importlib import import_module
    ops = import_module("simple-inference-autoresearch_amd._lib").gpu_ops()
    with pytest.raises(NotImplementedError, match="dtype"):   # the C ABI itself takes q's dtype or fp32
        ops.prefill_rope(q, k, v, cos, sin, False, None, 0, True, 0.1, False)
    torch.cuda.synchronize()


def test_graph_replays_at_new_device_positions(gpu_pkg):
    """The fused prefill reads its positions on the device: one captured graph serves every
    start position, and each replay equals the eager call."""
    B, Hq, Hkv, T, D = 2, 8, 2, 96, 128
    announce("rope prefill HIP-graph replay")
    q, k, v = inputs(B, Hq, Hkv, T, T, D, torch.bfloat16, seed=31)
    cos, sin = tables(512, D, torch.bfloat16)
    sp = torch.tensor([0, 0], dtype=torch.int32, device=DEV)
    gpu_pkg.rope_attention_flash_triton(q, k, v, cos, sin, causal=True, start_pos=sp)   # warm-up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = gpu_pkg.rope_attention_flash_triton(q, k, v, cos, sin, causal=True, start_pos=sp)
    for starts in ([0, 0], [5, 300], [17, 17], [400, 2]):
        sp.copy_(torch.tensor(starts, dtype=torch.int32))
        g.replay()
        torch.cuda.synchronize()
        want = gpu_pkg.rope_attention_flash_triton(q, k, v, cos, sin, causal=True,
                                                   start_pos=torch.tensor(starts, dtype=torch.int32, device=DEV))
        torch.cuda.synchronize()
        assert torch.equal(out, want), starts
        assert torch.equal(want, unfused(gpu_pkg, q, k, v, cos, sin, starts, False, True)), starts


def test_argument_errors(gpu_pkg):
    q, k, v = inputs(1, 4, 1, 32, 32, 64, torch.bfloat16, seed=2)
    cos, sin = tables(40, 64, torch.bfloat16)
    with pytest.raises(ValueError, match="positions"):
        gpu_pkg.rope_attention_flash_triton(q, k, v, cos, sin, causal=True, start_offset=10)   # rows 40, 41
    with pytest.raises(ValueError, match="identical shape"):
        gpu_pkg.rope_attention_flash_triton(q, k, v, cos, sin[:, :32], causal=True)
    with pytest.raises(NotImplementedError):
        gpu_pkg.rope_attention_flash_triton(q.float(), k.float(), v.float(), cos, sin, causal=True)
    torch.cuda.synchronize()
