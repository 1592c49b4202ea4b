"""GPU parity of the float32 attention path (BASELINE config 1 and fp32 callers).

The reference wrappers accept float32 tensors and return q's dtype
(kernels/flash_decode_kernel.py:119-160, kernels/attention_kernel.py:235-305);
its decode kernel computes in fp32 on vector lanes.  Float32 q or K/V run on
this library's fp32 vector-ALU kernel, so the bar is fp32 rounding: max-abs
<= 1e-5 against the float64 oracle for N(0,1) inputs (outputs are O(1)).
Calls that mix a 16-bit q with fp32 K/V return q's dtype and are held to the
16-bit bar (2e-3 before one output rounding).
"""

from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from oracle import attention as O
from helpers import announce, assert_close, f64

pytestmark = pytest.mark.gpu

syn = importlib.import_module("simple-inference-autoresearch_amd.synthetic")
DEV = "cuda"
FP32_TOL = 1e-5


def test_config1_decode(gpu_pkg):
    """B1, 32/8 heads, D64, ctx 512, fp32 N(0,1) (seed 0), scale 1/8,
    through attention_flash_decode and the eager module step gqa_attention."""
    announce("config 1: fp32 contiguous decode B1 32/8 D64 ctx 512")
    q, k, v = syn.cfg1()
    ref = O.gqa_decode(q.double().numpy(), k.double().numpy(), v.double().numpy(), 512, 1.0 / 8)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kl = torch.tensor([512], dtype=torch.int32, device=DEV)
    out = gpu_pkg.attention_flash_decode(qd, kd, vd, kl, 1.0 / 8)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and out.shape == (1, 1, 32, 64)
    assert_close(out, ref, FP32_TOL, "config 1 attention_flash_decode")
    step = gpu_pkg.gqa_attention(qd, kd, vd)
    torch.cuda.synchronize()
    assert step.shape == (1, 1, 32 * 64)
    assert_close(step.view(1, 1, 32, 64), ref, FP32_TOL, "config 1 gqa_attention")


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("G", [1, 4, 8, 12])
def test_fp32_contiguous(gpu_pkg, D, G):
    announce(f"fp32 contiguous decode D={D} G={G}")
    B, Hkv, S = 3, 2, 300
    g = torch.Generator(device=DEV).manual_seed(100 + D + G)
    q = torch.randn(B, G * Hkv, 1, D, generator=g, device=DEV)
    k = torch.randn(B, Hkv, S, D, generator=g, device=DEV)
    v = torch.randn(B, Hkv, S, D, generator=g, device=DEV)
    for lens in ([0, 1, 300], [300], [257, 13, 64]):
        kl = torch.tensor(lens, dtype=torch.int32, device=DEV)
        out = gpu_pkg.attention_flash_decode(q, k, v, kl)
        torch.cuda.synchronize()
        ref = O.gqa_decode(f64(q), f64(k), f64(v), lens)
        assert_close(out, ref, FP32_TOL, f"fp32 D={D} G={G} lens={lens}")


@pytest.mark.parametrize("tps", [0, 1, 2, 5, 64])
def test_fp32_split_invariance(gpu_pkg, tps):
    """Forced key-range splits (tiles of 16 keys) give the unsplit answer."""
    announce(f"fp32 decode forced split tiles_per_split={tps}")
    B, Hq, Hkv, S, D = 2, 16, 4, 1000, 128
    g = torch.Generator(device=DEV).manual_seed(7)
    q = torch.randn(B, Hq, 1, D, generator=g, device=DEV)
    k = torch.randn(B, Hkv, S, D, generator=g, device=DEV)
    v = torch.randn(B, Hkv, S, D, generator=g, device=DEV)
    lens = [1000, 517]
    kl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    with gpu_pkg.decode_options(tiles_per_split=tps):
        out = gpu_pkg.attention_flash_decode(q, k, v, kl)
    torch.cuda.synchronize()
    assert_close(out, O.gqa_decode(f64(q), f64(k), f64(v), lens), FP32_TOL, f"split {tps}")


def test_fp32_paged(gpu_pkg):
    announce("fp32 paged decode")
    ctx = [700, 1, 300, 1500, 16]
    case = syn.paged_case(ctx, Hq=16, Hkv=4, D=128, page=32, seed=11, device=DEV, kv="bf16",
                          q_dtype=torch.float32)
    kp, vp = case.k_pool.float(), case.v_pool.float()
    out = gpu_pkg.paged_attention_flash_decode(case.q, kp, vp, case.block_table, case.kv_len, 32)
    torch.cuda.synchronize()
    ref = O.paged_decode(f64(case.q), f64(kp), f64(vp), case.block_table.cpu().numpy(), ctx, 32)
    assert_close(out, ref, FP32_TOL, "fp32 paged")


@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.float16])
def test_fp32_query_int8_cache(gpu_pkg, scale_dtype):
    """fp32 q over an int8 cache (the int8 entry points, paged and contiguous)."""
    announce(f"fp32 q, int8 K/V, scales {scale_dtype}")
    ctx = [900, 33, 256]
    case = syn.paged_case(ctx, Hq=32, Hkv=8, D=128, page=16, seed=12, device=DEV, kv="int8",
                          q_dtype=torch.float32, scale_dtype=scale_dtype)
    out = gpu_pkg.paged_gqa_int8_flash_decode(case.q, case.k_pool, case.v_pool, case.k_scale, case.v_scale,
                                              case.block_table, case.kv_len, 16)
    torch.cuda.synchronize()
    ref = O.paged_int8_decode(f64(case.q), case.k_pool.cpu().numpy(), case.v_pool.cpu().numpy(),
                              f64(case.k_scale), f64(case.v_scale), case.block_table.cpu().numpy(), ctx, 16)
    assert_close(out, ref, FP32_TOL, "fp32 q int8 paged")
    # contiguous int8 views of the same data through the identity of a gathered cache
    B, Hkv, D = 3, 8, 128
    S = max(ctx)
    kc = torch.zeros(B, Hkv, S, D, dtype=torch.int8, device=DEV)
    vc = torch.zeros_like(kc)
    ksc = torch.zeros(B, Hkv, S, dtype=scale_dtype, device=DEV)
    vsc = torch.zeros_like(ksc)
    for b, n in enumerate(ctx):
        t = torch.arange(n, device=DEV)
        pg = case.block_table[b, t // 16].long()
        kc[b, :, :n] = case.k_pool[pg, :, t % 16].transpose(0, 1)
        vc[b, :, :n] = case.v_pool[pg, :, t % 16].transpose(0, 1)
        ksc[b, :, :n] = case.k_scale[pg, :, t % 16].transpose(0, 1)
        vsc[b, :, :n] = case.v_scale[pg, :, t % 16].transpose(0, 1)
    out2 = gpu_pkg.attention_flash_decode_int8(case.q, kc, vc, ksc, vsc, case.kv_len)
    torch.cuda.synchronize()
    assert_close(out2, ref, FP32_TOL, "fp32 q int8 contiguous")


@pytest.mark.parametrize("q_dtype", [torch.float16, torch.bfloat16])
def test_16bit_query_fp32_cache(gpu_pkg, q_dtype):
    """A 16-bit q over an fp32 cache returns q's dtype (16-bit bar)."""
    announce(f"{q_dtype} q, fp32 K/V")
    B, Hq, Hkv, S, D = 2, 8, 2, 200, 64
    g = torch.Generator(device=DEV).manual_seed(13)
    q = torch.randn(B, Hq, 1, D, generator=g, device=DEV).to(q_dtype)
    k = torch.randn(B, Hkv, S, D, generator=g, device=DEV)
    v = torch.randn(B, Hkv, S, D, generator=g, device=DEV)
    out = gpu_pkg.attention_flash_decode(q, k, v, torch.tensor([200, 77], dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert out.dtype == q_dtype
    assert_close(out, O.gqa_decode(f64(q), f64(k), f64(v), [200, 77]), 2e-3, "16-bit q fp32 K/V")


@pytest.mark.parametrize("D", [16, 64, 128, 256])
@pytest.mark.parametrize("Tq,Tk", [(37, 37), (5, 90), (9, 4), (1, 50)])
def test_fp32_prefill(gpu_pkg, D, Tq, Tk):
    """fp32 attention_flash_triton: causal with the bottom-right offset (Tq < Tk),
    fully masked leading rows (Tq > Tk) and the non-causal form."""
    announce(f"fp32 prefill D={D} Tq={Tq} Tk={Tk}")
    B, Hq, Hkv = 2, 8, 2
    g = torch.Generator(device=DEV).manual_seed(D + Tq + Tk)
    q = torch.randn(B, Hq, Tq, D, generator=g, device=DEV)
    k = torch.randn(B, Hkv, Tk, D, generator=g, device=DEV)
    v = torch.randn(B, Hkv, Tk, D, generator=g, device=DEV)
    for causal in (True, False):
        out = gpu_pkg.attention_flash_triton(q, k, v, causal=causal)
        tm = gpu_pkg.attention_flash_triton(q, k, v, causal=causal, out_token_major=True)
        torch.cuda.synchronize()
        ref = O.flash_attention(f64(q), f64(k), f64(v), causal)
        assert out.dtype == torch.float32
        assert_close(out, ref, FP32_TOL, f"fp32 prefill causal={causal}")
        assert_close(tm, ref.transpose(0, 2, 1, 3), FP32_TOL, f"fp32 prefill token-major causal={causal}")
