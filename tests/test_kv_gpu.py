"""GPU parity of the KV write path and the cache drop-ins against the CPU oracle.

Bars:
* int8 quantisation: bit-exact (codes and scales) against ``oracle.quantize_kv_int8``,
  the restatement of ``model/kv_cache.py:58-67`` pinned by the CPU suite;
* 16-bit / fp32 writes: bit-exact copies (or casts) at the oracle's positions;
* attention read back through the caches: the decode bars of ``test_decode_gpu``
  (2e-3 max-abs or one output ulp; int8 against attention over the dequantised cache).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import announce, assert_close, f64
from oracle import attention as O

pytestmark = pytest.mark.gpu
DEV = "cuda"

_NP_DT = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}


def close(got, ref, what, atol):
    assert_close(got, ref, atol, what)


def oracle_quant(x: torch.Tensor, scale_dtype: torch.dtype):
    xi, s = O.quantize_kv_int8(x.float().cpu().numpy(), _NP_DT[x.dtype],
                               "float16" if scale_dtype == torch.float16 else "float32")
    return xi, s


# ------------------------------------------------------------ quantize_kv_int8


@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(2, 3, 5, 128), (7, 64), (4, 2, 3, 256), (1, 1, 1, 16), (3, 32)])
@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_quantize_bit_exact(gpu_pkg, src, shape, scale_dtype):
    announce(f"quantize_kv_int8 {src} {shape} scale {scale_dtype}")
    g = torch.Generator(device=DEV).manual_seed(sum(shape) * 7 + len(str(src)))
    x = (torch.randn(shape, generator=g, device=DEV) * 3).to(src)
    x.view(-1, shape[-1])[0] = 0                 # an all-zero row: amax floor 1e-8
    xi, s = gpu_pkg.quantize_kv_int8(x, scale_dtype=scale_dtype)
    torch.cuda.synchronize()
    ri, rs = oracle_quant(x, scale_dtype)
    assert xi.dtype == torch.int8 and xi.shape == x.shape and s.shape == x.shape[:-1] and s.dtype == scale_dtype
    np.testing.assert_array_equal(xi.cpu().numpy(), ri)
    np.testing.assert_array_equal(s.float().cpu().numpy(), np.asarray(rs, dtype=np.float32))


def test_quantize_ties_round_half_even(gpu_pkg):
    """amax = 127 gives scale exactly 1, so x = k + 0.5 lands on a tie: half to even."""
    announce("quantize ties")
    row = torch.tensor([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5] + [0.0] * 8, device=DEV)
    xi, s = gpu_pkg.quantize_kv_int8(row.to(torch.bfloat16)[None])
    torch.cuda.synchronize()
    assert xi[0, :8].tolist() == [127, 0, 2, 2, 0, -2, -2, 126]
    assert s.float().item() == 1.0


def test_quantize_strided_view(gpu_pkg):
    announce("quantize strided view")
    base = torch.randn(4, 16, 3, 128, device=DEV).to(torch.bfloat16)
    x = base.transpose(1, 2)                      # (4, 3, 16, 128) view, head_dim contiguous
    xi, s = gpu_pkg.quantize_kv_int8(x)
    ri, rs = oracle_quant(x, torch.float16)
    np.testing.assert_array_equal(xi.cpu().numpy(), ri)
    np.testing.assert_array_equal(s.float().cpu().numpy(), np.asarray(rs, dtype=np.float32))


# ------------------------------------------------------------------- kv_write


@pytest.mark.parametrize("src,dst", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16),
                                     (torch.float16, torch.float16), (torch.bfloat16, torch.float32)])
def test_kv_write_contiguous_copy(gpu_pkg, src, dst):
    announce(f"kv_write contiguous {src}->{dst}")
    B, H, T, S, D = 3, 4, 5, 12, 128
    k = torch.randn(B, H, T, D, device=DEV).to(src)
    v = torch.randn(B, H, T, D, device=DEV).to(src)
    kc = torch.full((B + 1, H, S, D), 7.0, device=DEV).to(dst)
    vc = torch.full((B + 1, H, S, D), 7.0, device=DEV).to(dst)
    gpu_pkg.kv_write(k, v, kc, vc, start_offset=4)
    torch.cuda.synchronize()
    base = np.full((B, H, S, D), 7.0)
    np.testing.assert_array_equal(f64(kc)[:B], O.kv_write_contiguous(base, f64(k.to(dst)), 4))
    np.testing.assert_array_equal(f64(vc)[:B], O.kv_write_contiguous(base, f64(v.to(dst)), 4))
    assert (f64(kc)[B] == 7.0).all()             # the extra batch row is untouched


def test_kv_write_device_positions_and_bounds(gpu_pkg):
    """Per-sequence device start; positions past the cache are skipped, nothing else is touched."""
    announce("kv_write device positions")
    B, H, S, D = 4, 2, 6, 64
    k = torch.randn(B, H, 1, D, device=DEV).to(torch.bfloat16)
    pos = torch.tensor([0, 5, 6, 3], dtype=torch.int32, device=DEV)    # 6 is outside S
    kc = torch.zeros(B, H, S, D, dtype=torch.bfloat16, device=DEV)
    gpu_pkg.kv_write(k, None, kc, None, start_pos=pos)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(f64(kc), O.kv_write_contiguous(np.zeros((B, H, S, D)), f64(k), [0, 5, 6, 3]))


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_kv_write_contiguous_int8(gpu_pkg, scale_dtype):
    announce(f"kv_write contiguous int8 scales {scale_dtype}")
    B, H, T, S, D = 2, 8, 7, 16, 128
    k = torch.randn(B, H, T, D, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, H, T, D, device=DEV).to(torch.bfloat16)
    kc = torch.zeros(B, H, S, D, dtype=torch.int8, device=DEV)
    vc = torch.zeros_like(kc)
    ks = torch.zeros(B, H, S, dtype=scale_dtype, device=DEV)
    vs = torch.zeros_like(ks)
    gpu_pkg.kv_write(k, v, kc, vc, ks, vs, start_offset=9)
    torch.cuda.synchronize()
    for x, c, s in ((k, kc, ks), (v, vc, vs)):
        ri, rs = oracle_quant(x, scale_dtype)
        np.testing.assert_array_equal(c.cpu().numpy(), O.kv_write_contiguous(np.zeros((B, H, S, D), np.int8), ri, 9))
        want_s = O.kv_write_contiguous(np.zeros((B, H, S, 1), np.float32), np.asarray(rs, np.float32)[..., None], 9)
        np.testing.assert_array_equal(s.float().cpu().numpy(), want_s[..., 0])


@pytest.mark.parametrize("dst", [torch.float16, torch.int8])
@pytest.mark.parametrize("page", [16, 32])
def test_kv_write_paged(gpu_pkg, dst, page):
    announce(f"kv_write paged {dst} page {page}")
    B, H, T, D = 3, 4, 41, 128
    nblk = 3
    P = B * nblk + 2
    g = torch.Generator().manual_seed(7)
    bt = torch.randperm(P, generator=g)[:B * nblk].reshape(B, nblk).to(torch.int32)
    k = torch.randn(B, H, T, D, device=DEV).to(torch.float16)
    kp = torch.zeros(P, H, page, D, dtype=dst, device=DEV)
    ks = torch.zeros(P, H, page, dtype=torch.float32, device=DEV) if dst == torch.int8 else None
    start = torch.tensor([0, 3, 7], dtype=torch.int32, device=DEV)
    gpu_pkg.kv_write(k, None, kp, None, ks, None, block_table=bt.to(DEV), start_pos=start, page_size=page)
    torch.cuda.synchronize()
    if dst == torch.int8:
        ri, rs = oracle_quant(k, torch.float32)
        np.testing.assert_array_equal(kp.cpu().numpy(),
                                      O.kv_write_paged(np.zeros((P, H, page, D), np.int8), ri, bt.numpy(), page,
                                                       [0, 3, 7]))
        want_s = O.kv_write_paged(np.zeros((P, H, page, 1), np.float32), np.asarray(rs, np.float32)[..., None],
                                  bt.numpy(), page, [0, 3, 7])
        np.testing.assert_array_equal(ks.cpu().numpy(), want_s[..., 0])
    else:
        np.testing.assert_array_equal(f64(kp), O.kv_write_paged(np.zeros((P, H, page, D)), f64(k), bt.numpy(), page,
                                                                [0, 3, 7]))


# -------------------------------------------------------------- cache drop-ins


@pytest.mark.parametrize("max_seq", [64, 300])      # 300 > 256: the int8 cache of model/kv_cache.py
def test_kvcache_update_matches_reference_contract(gpu_pkg, max_seq):
    announce(f"KVCache.update max_seq {max_seq}")
    L, B, H, D = 2, 3, 2, 128
    cache = gpu_pkg.KVCache(L, 4, max_seq, H, D, dtype=torch.bfloat16, device=DEV)
    T = 20
    k = torch.randn(B, T, H, D, device=DEV).to(torch.bfloat16).transpose(1, 2)   # the reference's transposed views
    v = torch.randn(B, T, H, D, device=DEV).to(torch.bfloat16).transpose(1, 2)
    rk, rv = cache.update(1, 0, k, v)
    k2 = torch.randn(B, H, 1, D, device=DEV).to(torch.bfloat16)
    v2 = torch.randn(B, H, 1, D, device=DEV).to(torch.bfloat16)
    rk2, rv2 = cache.update(1, T, k2, v2)
    torch.cuda.synchronize()
    if not cache.is_int8:
        assert rk2.shape == (B, H, T + 1, D)
        assert torch.equal(rk2[:, :, :T], k) and torch.equal(rk2[:, :, T:], k2) and torch.equal(rv2[:, :, T:], v2)
    else:
        assert rk is k and rv2 is v2              # the int8 cache returns the new bf16 tensors
        kall = torch.cat([k, k2], 2)
        ri, rs = oracle_quant(kall, torch.float16)
        np.testing.assert_array_equal(cache.k_cache[1, :B, :, :T + 1].cpu().numpy(), ri)
        np.testing.assert_array_equal(cache.k_scale[1, :B, :, :T + 1].float().cpu().numpy(),
                                      np.asarray(rs, np.float32))
    assert not cache.k_cache[0].any()             # other layers untouched
    with pytest.raises(AssertionError):
        cache.update(0, max_seq - 1, k, v)        # overflow asserts like the reference


@pytest.mark.parametrize("max_seq", [96, 512])
def test_decode_step_attention_contiguous(gpu_pkg, max_seq):
    """The captured decode step: write at ctx.pos_index, attend over ctx.kv_len."""
    announce(f"decode_step_attention max_seq {max_seq}")
    B, Hq, H, D, T0 = 4, 32, 8, 128, 60
    cache = gpu_pkg.KVCache(1, B, max_seq, H, D, device=DEV)
    k0 = torch.randn(B, H, T0, D, device=DEV).to(torch.bfloat16)
    v0 = torch.randn(B, H, T0, D, device=DEV).to(torch.bfloat16)
    cache.update(0, 0, k0, v0)
    ctx = gpu_pkg.DecodeCtx(D, DEV)
    ks, vs = [k0], [v0]
    for step in range(3):
        q = torch.randn(B, Hq, 1, D, device=DEV).to(torch.bfloat16)
        kn = torch.randn(B, H, 1, D, device=DEV).to(torch.bfloat16)
        vn = torch.randn(B, H, 1, D, device=DEV).to(torch.bfloat16)
        ctx.set_position(T0 + step)
        out = gpu_pkg.decode_step_attention(q, kn, vn, cache, 0, ctx)
        torch.cuda.synchronize()
        ks.append(kn)
        vs.append(vn)
        kall, vall = torch.cat(ks, 2), torch.cat(vs, 2)
        if cache.is_int8:
            ki, ksc = oracle_quant(kall, torch.float16)
            vi, vsc = oracle_quant(vall, torch.float16)
            ref = O.int8_decode(f64(q), ki, vi, np.asarray(ksc, np.float64), np.asarray(vsc, np.float64), T0 + step + 1)
            close(out, ref, f"int8 step {step}", 1e-2)
            close(out, ref, f"int8 step {step} (tight)", 2e-3)
        else:
            close(out, O.gqa_decode(f64(q), f64(kall), f64(vall), T0 + step + 1), f"bf16 step {step}", 2e-3)


@pytest.mark.parametrize("kv_dtype", [None, torch.int8])
def test_paged_cache_prefill_then_decode(gpu_pkg, kv_dtype):
    """PagedKVCache: write_prefill, then decode steps whose slot comes from seq_lens on the device."""
    announce(f"PagedKVCache flow kv_dtype={kv_dtype}")
    B, Hq, H, D, T0, bs = 3, 16, 4, 128, 37, 16
    cache = gpu_pkg.PagedKVCache(2, 4, 100, H, D, block_size=bs, dtype=torch.bfloat16, device=DEV, kv_dtype=kv_dtype)
    k0 = torch.randn(B, H, T0, D, device=DEV).to(torch.bfloat16)
    v0 = torch.randn(B, H, T0, D, device=DEV).to(torch.bfloat16)
    cache.allocate(B, cache.max_blocks_per_seq)
    cache.write_prefill(1, B, k0, v0)
    cache.set_lengths(B, T0)
    ks, vs = [k0], [v0]
    for step in range(3):
        q = torch.randn(B, Hq, 1, D, device=DEV).to(torch.bfloat16)
        kn = torch.randn(B, H, 1, D, device=DEV).to(torch.bfloat16)
        vn = torch.randn(B, H, 1, D, device=DEV).to(torch.bfloat16)
        cache.begin_decode_step(B)
        cache.write_decode(1, kn, vn)
        out = cache.decode_attention(1, q)
        torch.cuda.synchronize()
        ks.append(kn)
        vs.append(vn)
        kall, vall = torch.cat(ks, 2), torch.cat(vs, 2)
        n = T0 + step + 1
        assert cache.seq_lens[:B].tolist() == [n] * B
        if cache.is_int8:
            ki, ksc = oracle_quant(kall, torch.float32)
            vi, vsc = oracle_quant(vall, torch.float32)
            ref = O.int8_decode(f64(q), ki, vi, np.asarray(ksc, np.float64), np.asarray(vsc, np.float64), n)
            close(out, ref, f"paged int8 step {step}", 2e-3)
        else:
            close(out, O.gqa_decode(f64(q), f64(kall), f64(vall), n), f"paged bf16 step {step}", 2e-3)
    assert not cache.k_pool[0].any()


def test_paged_decode_step_hip_graph(gpu_pkg):
    """begin_decode_step + write_decode + decode_attention captured once, replayed per step."""
    announce("PagedKVCache decode step in a HIP graph")
    B, Hq, H, D, T0, bs = 2, 32, 8, 128, 50, 16
    cache = gpu_pkg.PagedKVCache(1, B, 128, H, D, block_size=bs, device=DEV, kv_dtype=torch.int8)
    k0 = torch.randn(B, H, T0, D, device=DEV).to(torch.bfloat16)
    v0 = torch.randn(B, H, T0, D, device=DEV).to(torch.bfloat16)
    cache.allocate(B, cache.max_blocks_per_seq)
    cache.write_prefill(0, B, k0, v0)
    cache.set_lengths(B, T0)
    q = torch.zeros(B, Hq, 1, D, dtype=torch.bfloat16, device=DEV)
    kn = torch.zeros(B, H, 1, D, dtype=torch.bfloat16, device=DEV)
    vn = torch.zeros(B, H, 1, D, dtype=torch.bfloat16, device=DEV)

    def step():
        cache.begin_decode_step(B)
        cache.write_decode(0, kn, vn)
        return cache.decode_attention(0, q)

    # warm up (library load, workspace sizing) outside the capture, then rewind
    step()
    cache.set_lengths(B, T0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = step()
    torch.cuda.synchronize()
    cache.set_lengths(B, T0)                      # capture does not run the kernels; rewind anyway
    ks, vs = [k0], [v0]
    gen = torch.Generator(device=DEV).manual_seed(3)
    for i in range(4):
        q.copy_(torch.randn(B, Hq, 1, D, generator=gen, device=DEV))
        kn.copy_(torch.randn(B, H, 1, D, generator=gen, device=DEV))
        vn.copy_(torch.randn(B, H, 1, D, generator=gen, device=DEV))
        g.replay()
        torch.cuda.synchronize()
        ks.append(kn.clone())
        vs.append(vn.clone())
        n = T0 + i + 1
        assert cache.seq_lens[:B].tolist() == [n] * B
        ki, ksc = oracle_quant(torch.cat(ks, 2), torch.float32)
        vi, vsc = oracle_quant(torch.cat(vs, 2), torch.float32)
        ref = O.int8_decode(f64(q), ki, vi, np.asarray(ksc, np.float64), np.asarray(vsc, np.float64), n)
        close(out, ref, f"graph replay {i}", 2e-3)


# ------------------------------------------------------------------ attention step


@pytest.mark.parametrize("T,S", [(1, 77), (64, 64), (40, 100)])
def test_gqa_attention_eager_step(gpu_pkg, T, S):
    """ops/attention.py:311-345: causal for T > 1 (bottom-right), full for T == 1; (B, T, Hq*D) out."""
    announce(f"gqa_attention T={T} S={S}")
    B, Hq, H, D = 2, 8, 2, 128
    q = (torch.randn(B, T, Hq, D, device=DEV) * 0.5).to(torch.bfloat16).transpose(1, 2)
    k = (torch.randn(B, H, S, D, device=DEV) * 0.5).to(torch.bfloat16)
    v = (torch.randn(B, H, S, D, device=DEV) * 0.5).to(torch.bfloat16)
    out = gpu_pkg.gqa_attention(q, k, v)
    torch.cuda.synchronize()
    assert out.shape == (B, T, Hq * D)
    ref = O.flash_attention(f64(q), f64(k), f64(v), T > 1)               # (B, Hq, T, D)
    close(out.view(B, T, Hq, D).transpose(1, 2), ref, "gqa_attention", 2e-3)


def test_flash_triton_single_query_layouts(gpu_pkg):
    """Tq == 1 calls run on the decode kernels; both output layouts match the oracle."""
    announce("attention_flash_triton Tq=1")
    B, Hq, H, S, D = 3, 16, 4, 300, 64
    q = torch.randn(B, Hq, 1, D, device=DEV).to(torch.float16)
    k = torch.randn(B, H, S, D, device=DEV).to(torch.float16)
    v = torch.randn(B, H, S, D, device=DEV).to(torch.float16)
    ref = O.flash_attention(f64(q), f64(k), f64(v), True)
    a = gpu_pkg.attention_flash_triton(q, k, v, causal=True)
    b = gpu_pkg.attention_flash_triton(q, k, v, causal=False, out_token_major=True)
    torch.cuda.synchronize()
    assert a.shape == (B, Hq, 1, D) and b.shape == (B, 1, Hq, D)
    close(a, ref, "head-major", 2e-3)
    close(b.transpose(1, 2), ref, "token-major", 2e-3)


def test_kv_write_argument_errors(gpu_pkg):
    announce("kv_write argument errors")
    k = torch.zeros(2, 2, 3, 128, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(2, 2, 4, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        gpu_pkg.kv_write(k, None, kc, None, start_offset=2)            # positions 2..4 exceed S = 4
    with pytest.raises(ValueError):
        gpu_pkg.kv_write(k, None, kc.to(torch.int8), None)            # int8 destination without scales
    with pytest.raises(NotImplementedError):
        gpu_pkg.kv_write(k[..., :48], None, kc[..., :48], None)       # head_dim 48
    with pytest.raises(ValueError):
        gpu_pkg.kv_write(k, None, kc[:, :1], None)                    # head count mismatch
