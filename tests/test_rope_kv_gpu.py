"""GPU parity of the fused RoPE + KV write (``sia_rope_kv_write``).

Bar: bit-exact.  The expected result composes oracle functions that the CPU
suite pins on their own: ``oracle.rope.rope_qk`` at each token's table row,
rounding to k's dtype, ``oracle.attention.quantize_kv_int8`` for int8
destinations and ``kv_write_contiguous`` / ``kv_write_paged`` for the
scatter.  The fused launch must also equal the unfused sequence it replaces
on the GPU (``rope_triton`` then ``kv_write``; ``ops/attention.py:202-228``),
and the fused decode step (``rope_decode_step_attention``) must equal RoPE +
``decode_step_attention``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import announce
from oracle import attention as O
from oracle import rope as OR

pytestmark = pytest.mark.gpu
DEV = "cuda"
_NP_DT = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}


def host(t):
    return t.detach().float().cpu().numpy()


def tables(Tc, D, dtype, width=None, theta=10000.0):
    inv = 1.0 / theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = torch.outer(torch.arange(Tc, dtype=torch.float64), inv)
    c, s = ang.cos(), ang.sin()
    if (width or D) == D:
        c, s = torch.cat([c, c], -1), torch.cat([s, s], -1)
    return c.to(dtype).to(DEV), s.to(dtype).to(DEV)


def qkv_slices(B, T, Hq, Hkv, D, dtype, seed):
    """q, k, v as the token-major slices of one fused qkv buffer (ops/attention.py:172-177)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    qkv = torch.randn(B, T, (Hq + 2 * Hkv) * D, generator=g, device=DEV).to(dtype)
    q = qkv[..., :Hq * D].reshape(B, T, Hq, D)
    k = qkv[..., Hq * D:(Hq + Hkv) * D].reshape(B, T, Hkv, D)
    v = qkv[..., (Hq + Hkv) * D:].reshape(B, T, Hkv, D)
    return q, k, v


def expected_rotation(q, k, cos, sin, pos, interleaved):
    """Oracle q_rot, k_rot (B, T, H, D) with token (b, t) rotated by table row pos[b, t]."""
    B, T = pos.shape
    Tc = cos.shape[0]
    flat = pos.reshape(-1)
    valid = (flat >= 0) & (flat < Tc)
    rows = np.where(valid, flat, 0)
    c, s = host(cos)[rows], host(sin)[rows]
    dt = _NP_DT[k.dtype]
    qr = kr = None
    if q is not None:
        qr, _ = OR.rope_qk(host(q), host(k), c, s, interleaved=interleaved, dtype=dt)
        qr = qr * valid.reshape(B, T, 1, 1)           # rows outside the table: zeros
    _, kr = OR.rope_qk(host(k)[:, :, :1], host(k), c, s, interleaved=interleaved, dtype=dt)
    return qr, kr


def expected_cache(x_bthd, dst, scale_dtype, paged, block_table=None, page_size=0, start=0, offset=0,
                   src_dtype="bfloat16"):
    """Cache content after writing x (B, T, H, D) into zero-initialised dst (and scales)."""
    x = np.transpose(x_bthd, (0, 2, 1, 3))            # (B, H, T, D)
    if dst.dtype == torch.int8:
        xi, sc = O.quantize_kv_int8(x, src_dtype, "float16" if scale_dtype == torch.float16 else "float32")
        vals, scales = xi.astype(np.float64), sc.astype(np.float64)
    else:
        vals, scales = O.round_to_dtype(x, _NP_DT[dst.dtype]).astype(np.float64), None
    if paged:
        cache = O.kv_write_paged(np.zeros(tuple(dst.shape)), vals, block_table, page_size, start, offset)
        sc_out = None if scales is None else O.kv_write_paged(np.zeros(tuple(dst.shape[:3])), scales, block_table,
                                                              page_size, start, offset)
    else:
        cache = O.kv_write_contiguous(np.zeros(tuple(dst.shape)), vals, start, offset)
        sc_out = None if scales is None else O.kv_write_contiguous(np.zeros(tuple(dst.shape[:3])), scales, start,
                                                                   offset)
    return cache, sc_out


def assert_cache(dst, scale_dst, want, want_scales, what):
    got = dst.detach().cpu().to(torch.float64).numpy()
    assert np.array_equal(got, want), f"{what}: cache differs at {np.argwhere(got != want)[:4].tolist()}"
    if want_scales is not None:
        gs = scale_dst.detach().cpu().to(torch.float64).numpy()
        assert np.array_equal(gs, want_scales), f"{what}: scales differ"


@pytest.mark.parametrize("dst_dtype,scale_dtype", [(torch.int8, torch.float16), (torch.int8, torch.float32),
                                                   (torch.bfloat16, None)])
@pytest.mark.parametrize("interleaved", [False, True])
def test_contiguous_decode_per_sequence_positions(gpu_pkg, dst_dtype, scale_dtype, interleaved):
    B, Hq, Hkv, D, S = 5, 8, 2, 128, 40
    announce(f"rope_kv_write contiguous decode {dst_dtype} scale {scale_dtype} il={interleaved}")
    q, k, v = qkv_slices(B, 1, Hq, Hkv, D, torch.bfloat16, seed=1)
    cos, sin = tables(64, D, torch.bfloat16)
    start = torch.tensor([0, 7, 39, 40, 12], dtype=torch.int32, device=DEV)   # 40 is past the cache
    kc = torch.zeros(B, Hkv, S, D, dtype=dst_dtype, device=DEV)
    vc = torch.zeros_like(kc)
    ks = vs = None
    if dst_dtype == torch.int8:
        ks = torch.zeros(B, Hkv, S, dtype=scale_dtype, device=DEV)
        vs = torch.zeros_like(ks)
    qo = gpu_pkg.rope_kv_write(q, k, v, cos, sin, kc, vc, ks, vs, start_pos=start, interleaved=interleaved)
    torch.cuda.synchronize()
    pos = O.kv_write_positions(B, 1, start.cpu().numpy())
    qr, kr = expected_rotation(q, k, cos, sin, pos, interleaved)
    assert np.array_equal(host(qo), qr)
    for dst, sdst, x, what in ((kc, ks, kr, "k"), (vc, vs, host(v), "v")):
        want, want_s = expected_cache(x, dst, scale_dtype, False, start=start.cpu().numpy())
        assert_cache(dst, sdst, want, want_s, what)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float16, 256), (torch.float32, 32),
                                     (torch.bfloat16, 16)])
@pytest.mark.parametrize("interleaved", [False, True])
def test_contiguous_prefill_at_offset(gpu_pkg, dtype, D, interleaved):
    B, T, Hq, Hkv, S = 2, 7, 4, 2, 16
    announce(f"rope_kv_write prefill {dtype} D={D} il={interleaved}")
    q, k, v = qkv_slices(B, T, Hq, Hkv, D, dtype, seed=D)
    cos, sin = tables(S, D, torch.float32, width=D // 2)
    kc = torch.zeros(B, Hkv, S, D, dtype=dtype, device=DEV)
    vc = torch.zeros_like(kc)
    qo = gpu_pkg.rope_kv_write(q, k, v, cos, sin, kc, vc, start_offset=3, interleaved=interleaved)
    torch.cuda.synchronize()
    pos = O.kv_write_positions(B, T, 0, 3)
    qr, kr = expected_rotation(q, k, cos, sin, pos, interleaved)
    assert np.array_equal(host(qo), qr)
    want, _ = expected_cache(kr, kc, None, False, start=0, offset=3)
    assert_cache(kc, None, want, None, "k")
    want, _ = expected_cache(host(v), vc, None, False, start=0, offset=3)
    assert_cache(vc, None, want, None, "v")


def test_paged_int8_decode_llama3_tables(gpu_pkg):
    """The paged decode write of BASELINE config 3's layout: int8 pools, fp32 scales, position seq_lens - 1."""
    B, Hq, Hkv, D, page, nblk = 6, 32, 8, 128, 16, 9
    announce("rope_kv_write paged int8 decode")
    q, k, v = qkv_slices(B, 1, Hq, Hkv, D, torch.bfloat16, seed=3)
    rf = gpu_pkg.RopeFrequencies(D, nblk * page, device=torch.device(DEV))
    cos, sin = rf.get(nblk * page, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(5)
    perm = torch.randperm(B * nblk, generator=g).int()
    bt = perm.view(B, nblk).to(DEV)
    seq_lens = torch.tensor([1, 16, 17, 100, 144, 145], dtype=torch.int32, device=DEV)   # 145 > capacity
    kp = torch.zeros(B * nblk, Hkv, page, D, dtype=torch.int8, device=DEV)
    vp = torch.zeros_like(kp)
    ks = torch.zeros(B * nblk, Hkv, page, dtype=torch.float32, device=DEV)
    vs = torch.zeros_like(ks)
    qo = gpu_pkg.rope_kv_write(q, k, v, cos, sin, kp, vp, ks, vs, block_table=bt, start_pos=seq_lens,
                               start_offset=-1, page_size=page)
    torch.cuda.synchronize()
    pos = O.kv_write_positions(B, 1, seq_lens.cpu().numpy(), -1)
    qr, kr = expected_rotation(q, k, cos, sin, pos, False)
    assert np.array_equal(host(qo), qr)
    for dst, sdst, x, what in ((kp, ks, kr, "k"), (vp, vs, host(v), "v")):
        want, want_s = expected_cache(x, dst, torch.float32, True, bt.cpu().numpy(), page,
                                      seq_lens.cpu().numpy(), -1)
        assert_cache(dst, sdst, want, want_s, what)


def test_table_shorter_than_cache(gpu_pkg):
    """Positions past the table: K/V rows skipped, q rows zero."""
    B, Hq, Hkv, D, S = 3, 2, 1, 64, 20
    announce("rope_kv_write short table")
    q, k, v = qkv_slices(B, 1, Hq, Hkv, D, torch.bfloat16, seed=9)
    cos, sin = tables(10, D, torch.bfloat16)
    start = torch.tensor([2, 10, 15], dtype=torch.int32, device=DEV)
    kc = torch.zeros(B, Hkv, S, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    qo = gpu_pkg.rope_kv_write(q, k, v, cos, sin, kc, vc, start_pos=start)
    torch.cuda.synchronize()
    assert (host(qo)[1:] == 0).all()
    assert (host(kc)[1:] == 0).all() and (host(vc)[1:] == 0).all()
    pos = O.kv_write_positions(1, 1, [2])
    qr, kr = expected_rotation(q[:1], k[:1], cos, sin, pos, False)
    assert np.array_equal(host(qo)[:1], qr)
    assert np.array_equal(host(kc)[0, :, 2], kr[0, 0])
    assert np.array_equal(host(vc)[0, :, 2], host(v)[0, 0])


def test_k_only(gpu_pkg):
    announce("rope_kv_write k only")
    q, k, v = qkv_slices(2, 3, 4, 2, 128, torch.bfloat16, seed=4)
    cos, sin = tables(8, 128, torch.bfloat16)
    kc = torch.zeros(2, 2, 8, 128, dtype=torch.bfloat16, device=DEV)
    assert gpu_pkg.rope_kv_write(None, k, None, cos, sin, kc, None, start_offset=1) is None
    torch.cuda.synchronize()
    _, kr = expected_rotation(None, k, cos, sin, O.kv_write_positions(2, 3, 0, 1), False)
    want, _ = expected_cache(kr, kc, None, False, start=0, offset=1)
    assert_cache(kc, None, want, None, "k")


@pytest.mark.parametrize("int8", [False, True])
def test_fused_equals_unfused_sequence(gpu_pkg, int8):
    """One launch == rope_triton then kv_write (the reference's order, shared position)."""
    B, Hq, Hkv, D, S, p = 4, 32, 8, 128, 300, 257
    announce(f"rope_kv_write fused vs unfused int8={int8}")
    q, k, v = qkv_slices(B, 1, Hq, Hkv, D, torch.bfloat16, seed=7)
    rf = gpu_pkg.RopeFrequencies(D, S, device=torch.device(DEV))
    cos, sin = rf.get(S, dtype=torch.bfloat16)
    dst = torch.int8 if int8 else torch.bfloat16

    def caches():
        kc = torch.zeros(B, Hkv, S, D, dtype=dst, device=DEV)
        sc = torch.zeros(B, Hkv, S, dtype=torch.float16, device=DEV) if int8 else None
        return kc, torch.zeros_like(kc), sc, (torch.zeros_like(sc) if int8 else None)

    pos = torch.tensor([p], dtype=torch.int32, device=DEV)
    k1, v1, ks1, vs1 = caches()
    qo = gpu_pkg.rope_kv_write(q, k, v, cos, sin, k1, v1, ks1, vs1, start_pos=pos)
    k2, v2, ks2, vs2 = caches()
    qr, kr = gpu_pkg.rope_triton(q, k, cos[p:p + 1], sin[p:p + 1])
    gpu_pkg.kv_write(kr.transpose(1, 2), v.contiguous().transpose(1, 2), k2, v2, ks2, vs2, start_pos=pos)
    torch.cuda.synchronize()
    assert torch.equal(qo, qr)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    if int8:
        assert torch.equal(ks1, ks2) and torch.equal(vs1, vs2)


def test_rope_decode_step_attention(gpu_pkg):
    """The fused decode step == RoPE + decode_step_attention, int8 cache, per-sequence positions."""
    B, Hq, Hkv, D, S = 4, 32, 8, 128, 512
    announce("rope_decode_step_attention")
    torch.manual_seed(21)
    cache1 = gpu_pkg.KVCache(1, B, S, Hkv, D, device=DEV)
    cache2 = gpu_pkg.KVCache(1, B, S, Hkv, D, device=DEV)
    assert cache1.is_int8
    pre_k = torch.randn(B, Hkv, S, D, device=DEV).to(torch.bfloat16)
    pre_v = torch.randn(B, Hkv, S, D, device=DEV).to(torch.bfloat16)
    for c in (cache1, cache2):
        c.update(0, 0, pre_k, pre_v)
    rf = gpu_pkg.RopeFrequencies(D, S, device=torch.device(DEV))
    cos, sin = rf.get(S, dtype=torch.bfloat16)
    ctx = gpu_pkg.DecodeCtx(D, DEV, batch=B, per_sequence=True)
    ctx.set_position(torch.tensor([100, 300, 511, 7], dtype=torch.int32, device=DEV))
    q, k, v = qkv_slices(B, 1, Hq, Hkv, D, torch.bfloat16, seed=11)
    out1 = gpu_pkg.rope_decode_step_attention(q, k, v, cos, sin, cache1, 0, ctx)
    # unfused: per-sequence positions, so rotate each sequence with its own table row
    qr = torch.empty_like(q)
    kr = torch.empty_like(k)
    for b, p in enumerate([100, 300, 511, 7]):
        qb, kb = gpu_pkg.rope_triton(q[b:b + 1], k[b:b + 1], cos[p:p + 1], sin[p:p + 1])
        qr[b:b + 1], kr[b:b + 1] = qb, kb
    out2 = gpu_pkg.decode_step_attention(qr.transpose(1, 2), kr.transpose(1, 2), v.contiguous().transpose(1, 2),
                                         cache2, 0, ctx)
    torch.cuda.synchronize()
    assert torch.equal(cache1.k_cache, cache2.k_cache) and torch.equal(cache1.k_scale, cache2.k_scale)
    assert torch.equal(cache1.v_cache, cache2.v_cache)
    assert torch.equal(out1, out2)


def test_paged_cache_write_decode_rope(gpu_pkg):
    B, Hq, Hkv, D = 3, 16, 4, 128
    announce("PagedKVCache.write_decode_rope")
    cache = gpu_pkg.PagedKVCache(1, B, 64, Hkv, D, block_size=16, kv_dtype=torch.int8, device=DEV)
    cache.allocate(B, 4)
    cache.set_lengths(B, 20)
    cache.begin_decode_step(B)
    rf = gpu_pkg.RopeFrequencies(D, 64, device=torch.device(DEV))
    cos, sin = rf.get(64, dtype=torch.bfloat16)
    q, k, v = qkv_slices(B, 1, Hq, Hkv, D, torch.bfloat16, seed=13)
    qo = cache.write_decode_rope(0, q, k, v, cos, sin)
    torch.cuda.synchronize()
    qr, kr = gpu_pkg.rope_triton(q, k, cos[20:21], sin[20:21])
    assert torch.equal(qo, qr)
    kp, vp, ks, vs = cache.layer(0)
    bt = cache.block_tables[:B].cpu().numpy()
    xi, sc = O.quantize_kv_int8(np.transpose(host(kr), (0, 2, 1, 3)), "bfloat16", "float32")
    for b in range(B):
        pg = int(bt[b, 20 // 16])
        assert np.array_equal(kp[pg, :, 20 % 16].cpu().numpy(), xi[b, :, 0])
        assert np.array_equal(ks[pg, :, 20 % 16].cpu().numpy(), sc[b, :, 0])


def test_invalid_arguments(gpu_pkg):
    q, k, v = qkv_slices(1, 1, 2, 1, 64, torch.bfloat16, seed=1)
    cos, sin = tables(4, 64, torch.bfloat16)
    kc = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="identical shape"):
        gpu_pkg.rope_kv_write(q, k, v, cos, sin[:3], kc, torch.zeros_like(kc))
    with pytest.raises(ValueError, match="head_dim"):
        gpu_pkg.rope_kv_write(q, k, v, cos[:, :20], sin[:, :20], kc, torch.zeros_like(kc))
    with pytest.raises(ValueError, match="share a dtype"):
        gpu_pkg.rope_kv_write(q.float(), k, v, cos, sin, kc, torch.zeros_like(kc))
    # host-known positions past the 4-row tables are an error (nothing written)
    kc8 = torch.zeros(1, 1, 8, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="rows"):
        gpu_pkg.rope_kv_write(q, k, v, cos, sin, kc8, torch.zeros_like(kc8), start_offset=4)
    torch.cuda.synchronize()
    assert not kc8.any()


def test_no_tokens(gpu_pkg):
    """Zero tokens (T = 0, empty tensors without a data pointer): RoPE returns
    empty rotations, the cache writes leave the cache untouched and the int8
    quantiser returns empty outputs, as the reference's empty grids and
    tensor ops do."""
    announce("rope / kv write / quantise with no tokens")
    q, k, v = qkv_slices(2, 0, 4, 2, 64, torch.bfloat16, seed=2)
    cos, sin = tables(8, 64, torch.bfloat16)
    qr, kr = gpu_pkg.rope_triton(q, k, cos, sin)
    assert qr.shape == q.shape and kr.shape == k.shape
    kc = torch.full((2, 2, 8, 64), 7.0, dtype=torch.bfloat16, device=DEV)
    vc = kc.clone()
    qo = gpu_pkg.rope_kv_write(q, k, v, cos, sin, kc, vc, start_offset=3)
    assert qo.shape == q.shape
    gpu_pkg.kv_write(k.transpose(1, 2), v.transpose(1, 2), kc, vc)
    xi, sc = gpu_pkg.quantize_kv_int8(torch.empty(0, 2, 64, dtype=torch.bfloat16, device=DEV))
    torch.cuda.synchronize()
    assert torch.all(kc == 7.0) and torch.all(vc == 7.0)
    assert xi.shape == (0, 2, 64) and xi.dtype == torch.int8 and sc.shape == (0, 2)


def test_rope_decode_step_hip_graph_contiguous(gpu_pkg):
    """ops/attention.py:180-245 as one captured graph: fused RoPE + int8 write + attention,
    replayed at new per-sequence positions (ctx filled between replays, as
    model/cuda_graph_decode.py:98-102 does); every replay equals the eager unfused step."""
    B, Hq, Hkv, D, S = 3, 32, 8, 128, 600
    announce("rope_decode_step_attention in a HIP graph (contiguous int8 cache)")
    torch.manual_seed(31)
    cg = gpu_pkg.KVCache(1, B, S, Hkv, D, device=DEV)
    ce = gpu_pkg.KVCache(1, B, S, Hkv, D, device=DEV)
    pre_k = torch.randn(B, Hkv, S, D, device=DEV).to(torch.bfloat16)
    pre_v = torch.randn(B, Hkv, S, D, device=DEV).to(torch.bfloat16)
    for c in (cg, ce):
        c.update(0, 0, pre_k, pre_v)
    rf = gpu_pkg.RopeFrequencies(D, S, device=torch.device(DEV))
    cos, sin = rf.get(S, dtype=torch.bfloat16)
    ctx = gpu_pkg.DecodeCtx(D, DEV, batch=B, per_sequence=True)
    qkv = torch.zeros(B, 1, (Hq + 2 * Hkv) * D, dtype=torch.bfloat16, device=DEV)
    q = qkv[..., :Hq * D].view(B, 1, Hq, D)
    k = qkv[..., Hq * D:(Hq + Hkv) * D].view(B, 1, Hkv, D)
    v = qkv[..., (Hq + Hkv) * D:].view(B, 1, Hkv, D)
    ctx.set_position(torch.tensor([10, 20, 30], dtype=torch.int32, device=DEV))
    gpu_pkg.rope_decode_step_attention(q, k, v, cos, sin, cg, 0, ctx)      # warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = gpu_pkg.rope_decode_step_attention(q, k, v, cos, sin, cg, 0, ctx)
    torch.cuda.synchronize()
    gen = torch.Generator(device=DEV).manual_seed(5)
    for i, pos in enumerate(([10, 20, 30], [11, 200, 31], [12, 201, 599], [400, 7, 0])):
        pt = torch.tensor(pos, dtype=torch.int32, device=DEV)
        ctx.set_position(pt)
        qkv.copy_(torch.randn(qkv.shape, generator=gen, device=DEV))
        g.replay()
        torch.cuda.synchronize()
        # eager, unfused: per-sequence RoPE with the reference kernel's interface, then write + attend
        qr = torch.empty_like(q)
        kr = torch.empty_like(k)
        for b, p in enumerate(pos):
            qr[b:b + 1], kr[b:b + 1] = gpu_pkg.rope_triton(q[b:b + 1], k[b:b + 1], cos[p:p + 1], sin[p:p + 1])
        ref = gpu_pkg.decode_step_attention(qr.transpose(1, 2), kr.transpose(1, 2), v.contiguous().transpose(1, 2),
                                            ce, 0, ctx)
        torch.cuda.synchronize()
        assert torch.equal(cg.k_cache, ce.k_cache) and torch.equal(cg.v_cache, ce.v_cache), f"replay {i}"
        assert torch.equal(cg.k_scale, ce.k_scale) and torch.equal(cg.v_scale, ce.v_scale), f"replay {i}"
        assert torch.equal(out, ref), f"replay {i}"


def test_rope_paged_decode_step_hip_graph(gpu_pkg):
    """Paged pools with per-sequence seq_lens: begin_decode_step + write_decode_rope +
    decode_attention captured once and replayed; each replay equals the eager unfused step."""
    B, Hq, Hkv, D, bs = 3, 16, 4, 128, 16
    announce("paged rope decode step in a HIP graph")
    torch.manual_seed(41)
    caches = [gpu_pkg.PagedKVCache(1, B, 256, Hkv, D, block_size=bs, device=DEV, kv_dtype=torch.int8)
              for _ in range(2)]
    k0 = torch.randn(B, Hkv, 100, D, device=DEV).to(torch.bfloat16)
    v0 = torch.randn(B, Hkv, 100, D, device=DEV).to(torch.bfloat16)
    for c in caches:
        c.allocate(B, c.max_blocks_per_seq)
        c.write_prefill(0, B, k0, v0)
    lens0 = torch.tensor([5, 50, 100], dtype=torch.int32, device=DEV)
    rf = gpu_pkg.RopeFrequencies(D, 256, device=torch.device(DEV))
    cos, sin = rf.get(256, dtype=torch.bfloat16)
    q = torch.zeros(B, 1, Hq, D, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(B, 1, Hkv, D, dtype=torch.bfloat16, device=DEV)
    v = torch.zeros(B, 1, Hkv, D, dtype=torch.bfloat16, device=DEV)
    cg, ce = caches

    def step():
        cg.begin_decode_step(B)
        q_rot = cg.write_decode_rope(0, q, k, v, cos, sin)
        return cg.decode_attention(0, q_rot.transpose(1, 2))

    cg.seq_lens[:B].copy_(lens0)
    step()                                        # warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = step()
    torch.cuda.synchronize()
    cg.seq_lens[:B].copy_(lens0)
    ce.seq_lens[:B].copy_(lens0)
    gen = torch.Generator(device=DEV).manual_seed(6)
    for i in range(4):
        q.copy_(torch.randn(q.shape, generator=gen, device=DEV))
        k.copy_(torch.randn(k.shape, generator=gen, device=DEV))
        v.copy_(torch.randn(v.shape, generator=gen, device=DEV))
        g.replay()
        torch.cuda.synchronize()
        ce.begin_decode_step(B)
        pos = [int(n) - 1 for n in ce.seq_lens[:B].tolist()]
        qr = torch.empty_like(q)
        kr = torch.empty_like(k)
        for b, p in enumerate(pos):
            qr[b:b + 1], kr[b:b + 1] = gpu_pkg.rope_triton(q[b:b + 1], k[b:b + 1], cos[p:p + 1], sin[p:p + 1])
        ce.write_decode(0, kr.transpose(1, 2), v.transpose(1, 2))
        ref = ce.decode_attention(0, qr.transpose(1, 2))
        torch.cuda.synchronize()
        assert cg.seq_lens[:B].tolist() == ce.seq_lens[:B].tolist() == [n + i + 1 for n in (5, 50, 100)]
        assert torch.equal(cg.k_pool, ce.k_pool) and torch.equal(cg.k_scale_pool, ce.k_scale_pool), f"replay {i}"
        assert torch.equal(cg.v_pool, ce.v_pool), f"replay {i}"
        assert torch.equal(out, ref), f"replay {i}"
