"""GPU parity of the prefill kernel (attention_flash_triton) against the float64 oracle.

Tolerance: max-abs <= 2e-3 against the oracle before one rounding to the
output dtype, |got - ref| <= 2e-3 + 1/2 ulp(|ref| + 2e-3).  The PV product
uses f16 P and V (the reference rounds P to the input dtype; bf16 P alone
would exceed 2e-3 on rows with few keys).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import allowed_error, announce, assert_close, f64
from oracle import attention as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def check(out, ref, what, atol=2e-3):
    return assert_close(out, ref, atol, what)


def qkv(B, Hq, Hkv, Tq, Tk, D, dtype, seed, scale=0.5):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = (torch.randn(B, Hq, Tq, D, generator=g, device=DEV) * scale).to(dtype)
    k = (torch.randn(B, Hkv, Tk, D, generator=g, device=DEV) * scale).to(dtype)
    v = (torch.randn(B, Hkv, Tk, D, generator=g, device=DEV) * scale).to(dtype)
    return q, k, v


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [1, 17, 128, 130, 300])
@pytest.mark.parametrize("causal", [True, False])
def test_self_attention(gpu_pkg, D, dtype, T, causal):
    announce(f"prefill D={D} {dtype} T={T} causal={causal}")
    q, k, v = qkv(2, 8, 2, T, T, D, dtype, seed=T + D)
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=causal)
    torch.cuda.synchronize()
    check(out, O.flash_attention(f64(q), f64(k), f64(v), causal), f"D={D} T={T}")


@pytest.mark.parametrize("Tq,Tk", [(1, 700), (64, 300), (200, 513), (100, 64), (3, 1)])
def test_offset_causal(gpu_pkg, Tq, Tk):
    """Chunked prefill (Tq < Tk) and Tq > Tk, where leading rows see nothing."""
    announce(f"prefill offsets Tq={Tq} Tk={Tk}")
    q, k, v = qkv(1, 8, 2, Tq, Tk, 128, torch.bfloat16, seed=Tq * 7 + Tk)
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=True)
    torch.cuda.synchronize()
    ref = O.flash_attention(f64(q), f64(k), f64(v), True)
    check(out, ref, f"Tq={Tq} Tk={Tk}")
    if Tq > Tk:
        assert torch.all(out[:, :, :Tq - Tk] == 0)


@pytest.mark.parametrize("Tq,Tk", [(300, 300), (37, 421), (129, 64)])
def test_qwen_shape_d256(gpu_pkg, Tq, Tk):
    """Qwen3.5 full-attention layers: head_dim 256, 16 query / 4 KV heads (model/qwen35_plugin.py)."""
    announce(f"prefill D=256 Qwen shape Tq={Tq} Tk={Tk}")
    q, k, v = qkv(1, 16, 4, Tq, Tk, 256, torch.bfloat16, seed=Tq + Tk)
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=True, out_token_major=True)
    torch.cuda.synchronize()
    check(out.transpose(1, 2), O.flash_attention(f64(q), f64(k), f64(v), True), f"D=256 Tq={Tq} Tk={Tk}")


def test_strided_views_and_token_major(gpu_pkg):
    """The model passes transposed (B,T,H,D) views and wants token-major output."""
    announce("prefill strided views / token-major output")
    B, T, Hq, Hkv, D = 2, 200, 32, 8, 128
    g = torch.Generator(device=DEV).manual_seed(3)
    qt = (torch.randn(B, T, Hq, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    kt = (torch.randn(B, T, Hkv, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    vt = (torch.randn(B, T, Hkv, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    q, k, v = qt.transpose(1, 2), kt.transpose(1, 2), vt.transpose(1, 2)
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=True, assume_contiguous=True, out_token_major=True)
    ref_layout = gpu_pkg.attention_flash_triton(q.contiguous(), k.contiguous(), v.contiguous(), causal=True)
    torch.cuda.synchronize()
    assert out.shape == (B, T, Hq, D)
    assert torch.equal(out.transpose(1, 2), ref_layout)
    check(ref_layout, O.flash_attention(f64(q), f64(k), f64(v), True), "strided")


@pytest.mark.parametrize("layout", ["d_strided", "misaligned", "far_rows"])
def test_views_that_are_copied(gpu_pkg, layout):
    """Views the kernels cannot read in place are copied by the extension first:
    head_dim not contiguous, rows not 16-byte aligned, or K/V rows 32 MB apart
    (the rows of one 64-key block would span 2^31 bytes of 32-bit offsets).
    Each gives the same bits as the contiguous inputs, and matches the oracle."""
    announce(f"prefill views copied by the extension: {layout}")
    B, Hq, Hkv, T, D = (1, 4, 1, 70, 64) if layout == "far_rows" else (1, 8, 2, 100, 64)
    q, k, v = qkv(B, Hq, Hkv, T, T, D, torch.bfloat16, seed=17)
    if layout == "d_strided":        # (B, H, D, T) storage, transposed: head_dim has stride T
        views = [t.transpose(-1, -2).contiguous().transpose(-1, -2) for t in (q, k, v)]
    elif layout == "misaligned":     # rows start 2 bytes past a 16-byte boundary
        views = []
        for t in (q, k, v):
            base = torch.empty(*t.shape[:-1], D + 1, dtype=t.dtype, device=DEV)
            base[..., 1:] = t
            views.append(base[..., 1:])
    else:                            # one KV head, rows 2^24 elements (32 MB) apart
        row = 1 << 24
        views = [q]
        for t in (k, v):
            base = torch.empty(T * row, dtype=t.dtype, device=DEV)
            view = base.as_strided((B, Hkv, T, D), (0, 0, row, 1))
            view.copy_(t)
            views.append(view)
    out = gpu_pkg.attention_flash_triton(*views, causal=True)
    ref_layout = gpu_pkg.attention_flash_triton(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_layout)
    check(out, O.flash_attention(f64(q), f64(k), f64(v), True), layout)


@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (8, 4), (12, 4), (6, 1), (8, 1), (32, 2), (24, 2)])
@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("B,causal", [(1, True), (3, False), (2, True)])
def test_head_groupings(gpu_pkg, Hq, Hkv, D, B, causal):
    """Work-groups span the query heads of one KV head (powers of two dividing G):
    MHA, G = 2, 3, 4, 6, 8, 12 and 16, one or several head groups per KV head,
    batches whose unit count is or is not a multiple of 8 (XCD-aware order or not)."""
    announce(f"prefill heads {Hq}/{Hkv} D={D} B={B} causal={causal}")
    Tq, Tk = (130, 130) if causal else (97, 230)
    q, k, v = qkv(B, Hq, Hkv, Tq, Tk, D, torch.bfloat16, seed=Hq * 31 + Hkv * 7 + D + B)
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=causal)
    torch.cuda.synchronize()
    check(out, O.flash_attention(f64(q), f64(k), f64(v), causal), f"{Hq}/{Hkv} D={D} B={B}")


def test_gqa_mapping(gpu_pkg):
    """Each query head reads KV head hq // G: give each KV head a constant V."""
    announce("prefill GQA mapping")
    B, T, Hq, Hkv, D = 1, 64, 8, 2, 64
    q, k, _ = qkv(B, Hq, Hkv, T, T, D, torch.bfloat16, seed=5)
    v = torch.zeros(B, Hkv, T, D, dtype=torch.bfloat16, device=DEV)
    v[:, 0] = 1.0
    v[:, 1] = 2.0
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=True)
    torch.cuda.synchronize()
    for hq in range(Hq):
        assert torch.all(out[0, hq] == (1.0 if hq < 4 else 2.0)), hq


def check_every_head(out, q, k, v, causal, what):
    """Every (b, hq) of ``out`` (B, Hq, Tq, D) against the float64 oracle, one
    KV head's query group at a time (the host holds one group's scores)."""
    B, Hq = q.shape[0], q.shape[1]
    Hkv = k.shape[1]
    G = Hq // Hkv
    qf, kf, vf, of = f64(q), f64(k), f64(v), f64(out)
    worst = 0.0
    for b in range(B):
        for h in range(Hkv):
            ref = O.flash_attention(qf[b:b + 1, h * G:(h + 1) * G], kf[b:b + 1, h:h + 1], vf[b:b + 1, h:h + 1],
                                    causal)
            worst = max(worst, assert_close(of[b:b + 1, h * G:(h + 1) * G], ref, 2e-3, f"{what} b={b} hkv={h}",
                                            dtype=out.dtype))
        print(f"{what}: sequence {b} checked, max abs err so far {worst:.3e}", flush=True)
    return worst


def test_cfg4_full_size(gpu_pkg):
    """BASELINE config 4 (B4, T2048, 32/8 heads, D128, bf16, causal): every
    output head against the oracle."""
    announce("prefill config 4 full size")
    from importlib import import_module
    syn = import_module("simple-inference-autoresearch_amd.synthetic")
    q, k, v = syn.cfg4(DEV)
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=True)
    torch.cuda.synchronize()
    worst = check_every_head(out, q, k, v, True, "cfg4")
    print(f"cfg4 max abs err over all 128 heads: {worst:.3e}")


@pytest.mark.parametrize("B,Tq,Tk,causal", [(2, 2100, 2100, True), (4, 600, 2500, True), (2, 1500, 1700, False),
                                            (1, 2048, 2048, True), (1, 1500, 1700, False)])
def test_d128_grid_sizes(gpu_pkg, B, Tq, Tk, causal):
    """head_dim 128 runs 8-wave work-groups when the grid of them exceeds the
    CU count (the first three shapes; the small shapes of the other tests run
    4-wave groups).  One sequence of 2048 or 1500 rows runs 4-wave groups,
    more than one per CU and at most two: their order is folded so that each
    CU holds a heavy and a light one.  Ragged and offset lengths, every head
    against the oracle."""
    announce(f"prefill D=128 B={B} Tq={Tq} Tk={Tk} causal={causal}")
    g = torch.Generator(device=DEV).manual_seed(Tq + Tk)
    q = (torch.randn(B, 32, Tq, 128, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    k = (torch.randn(B, 8, Tk, 128, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    v = (torch.randn(B, 8, Tk, 128, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=causal)
    torch.cuda.synchronize()
    check_every_head(out, q, k, v, causal, f"B={B} Tq={Tq} Tk={Tk}")


@pytest.mark.parametrize("causal", [True, False])
def test_folded_order_without_xcd_remap(gpu_pkg, causal):
    """A folded 4-wave grid whose unit count (6) is not a multiple of 8, so the
    work-groups are folded in linear order rather than per XCD: one sequence
    of 1500 rows at 24/6 heads (282 work-groups), every head against the oracle."""
    announce(f"prefill folded linear order causal={causal}")
    q, k, v = qkv(1, 24, 6, 1500, 1500, 128, torch.bfloat16, seed=77 + causal)
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=causal)
    torch.cuda.synchronize()
    check_every_head(out, q, k, v, causal, "24/6 T=1500")


@pytest.mark.parametrize("B,Tq,Tk,causal,token_major", [(2, 1100, 1100, True, True), (2, 1100, 1100, False, False),
                                                         (3, 700, 1000, True, False), (1, 1000, 777, False, True),
                                                         (1, 130, 130, True, True)])
def test_f16_raw_v_rows(gpu_pkg, B, Tq, Tk, causal, token_major):
    """float16 at head_dim 128 reads raw V rows with transposed LDS reads (no
    V^T images, no repack launch), on the 8-wave grid (2 x 1100 rows: 288
    work-groups) and the 4-wave ones: ragged last key blocks, Tq != Tk, and
    token-major (B, T, H, D) storage read in place; every head against the
    oracle."""
    announce(f"prefill f16 raw V B={B} Tq={Tq} Tk={Tk} causal={causal} token_major={token_major}")
    q, k, v = qkv(B, 32, 8, Tq, Tk, 128, torch.float16, seed=Tq + 7 * Tk + causal)
    if token_major:
        q, k, v = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v))
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=causal)
    torch.cuda.synchronize()
    check_every_head(out, q, k, v, causal, f"f16 raw V Tq={Tq} Tk={Tk}")


@pytest.mark.parametrize("D,B,T,causal", [(128, 8, 256, True), (64, 4, 512, True), (32, 4, 512, False),
                                           (64, 1, 768, True), (32, 1, 769, True)])
def test_short_keys_two_groups_per_cu(gpu_pkg, D, B, T, causal):
    """bf16 variant 2 (V converted in LDS, no repack) on a grid of about two
    work-groups per CU (32/8 heads), and at D <= 64 on both sides of its
    768-key cut-over: every head against the oracle."""
    announce(f"prefill short keys, large grid D={D} B={B} T={T} causal={causal}")
    q, k, v = qkv(B, 32, 8, T, T, D, torch.bfloat16, seed=D + B + T)
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=causal)
    torch.cuda.synchronize()
    check_every_head(out, q, k, v, causal, f"D={D} B={B} T={T}")


@pytest.mark.parametrize("D", [32, 128])
def test_f16_needs_no_workspace(gpu_pkg, D):
    """Through the C ABI: float16 V read in place takes no workspace (NULL, 0),
    and gives the bits of the extension's call; bfloat16 still asks for one."""
    import ctypes
    from importlib import import_module
    lm = import_module("simple-inference-autoresearch_amd._lib")
    lib = lm.load_library()
    announce(f"prefill f16 without workspace D={D}")
    q, k, v = qkv(2, 16, 4, 300, 300, D, torch.float16, seed=D + 5)
    ref = gpu_pkg.attention_flash_triton(q, k, v, causal=True)
    out = torch.full_like(ref, float("nan"))
    dq, dk, dv, do = (lm.desc(t) for t in (q, k, v, out))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.sia_attention_flash_fwd(ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv), 1,
                                     ctypes.c_float(1.0 / (D ** 0.5)), ctypes.byref(do), None, 0, stream)
    torch.cuda.synchronize()
    assert rc == 0, lib.sia_last_error_message()
    assert torch.equal(out, ref)
    qb, kb, vb = (t.to(torch.bfloat16) for t in (q, k, v))
    ob = torch.empty_like(qb)
    dq, dk, dv, do = (lm.desc(t) for t in (qb, kb, vb, ob))
    rc = lib.sia_attention_flash_fwd(ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv), 1,
                                     ctypes.c_float(1.0 / (D ** 0.5)), ctypes.byref(do), None, 0, stream)
    assert rc == -3   # SIA_ERR_WORKSPACE: bfloat16 V is repacked into the workspace


@pytest.mark.parametrize("D", [32, 64])
@pytest.mark.parametrize("B,Hq,Hkv,Tq,Tk,causal,token_major", [(2, 32, 8, 900, 900, True, True),
                                                                (1, 16, 16, 333, 1001, False, True),
                                                                (3, 8, 2, 700, 513, True, False)])
def test_f16_raw_v_rows_small_head_dims(gpu_pkg, D, B, Hq, Hkv, Tq, Tk, causal, token_major):
    """float16 raw V rows and transposed reads at head_dim 32 and 64 (their
    own V-row swizzles; 16 and 8 rows per 1 KB transfer): ragged key blocks,
    Tq != Tk, token-major storage read in place, MHA and GQA, every head
    against the oracle."""
    announce(f"prefill f16 raw V D={D} B={B} {Hq}/{Hkv} Tq={Tq} Tk={Tk} causal={causal}")
    q, k, v = qkv(B, Hq, Hkv, Tq, Tk, D, torch.float16, seed=D + Tq + Tk)
    if token_major:
        q, k, v = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v))
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=causal)
    torch.cuda.synchronize()
    check_every_head(out, q, k, v, causal, f"f16 raw V D={D} Tq={Tq} Tk={Tk}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Tq,Tk,causal,token_major", [(256, 256, True, False), (512, 512, True, True),
                                                       (513, 513, True, True),
                                                       (40, 256, True, True), (256, 256, False, True),
                                                       (200, 255, False, False), (300, 64, True, False)])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_short_key_ranges(gpu_pkg, D, dtype, Tq, Tk, causal, token_major):
    """head_dim 32, 64 and 128 with at most 512 keys on a small grid: with bfloat16 each
    work-group converts its raw V blocks to f16 in LDS and reads them with
    transposed reads (no separate repack launch); 513 keys and up take the
    repack (float16 reads raw V rows at every length).  Both sides of
    the cut-over, chunked rows (Tq < Tk), Tq > Tk, and K/V read in place
    from token-major (B, T, H, D) storage, every head against the oracle."""
    announce(f"prefill short key range D={D} {dtype} Tq={Tq} Tk={Tk} causal={causal} token_major={token_major}")
    q, k, v = qkv(2, 16, 4, Tq, Tk, D, dtype, seed=Tq * 3 + Tk + D)
    if token_major:   # (B, T, H, D) storage seen as (B, H, T, D): row stride H*D elements
        q, k, v = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v))
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=causal)
    torch.cuda.synchronize()
    check_every_head(out, q, k, v, causal, f"Tq={Tq} Tk={Tk}")
    if causal and Tq > Tk:
        assert torch.all(out[:, :, :Tq - Tk] == 0)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_empty_lengths(gpu_pkg, D, dtype):
    """No keys: every row sees nothing and is written as zeros, the
    reference's guard of a fully masked row (kernels/attention_kernel.py:224-226).
    No queries: an empty output, token-major or not.  (Empty tensors may
    carry no data pointer.)"""
    announce(f"prefill empty lengths D={D} {dtype}")
    q, k, v = qkv(2, 8, 2, 5, 0, D, dtype, seed=3)
    for causal in (True, False):
        out = gpu_pkg.attention_flash_triton(q, k, v, causal=causal)
        torch.cuda.synchronize()
        assert out.shape == (2, 8, 5, D)
        assert torch.all(out == 0)
    q, k, v = qkv(2, 8, 2, 0, 7, D, dtype, seed=4)
    for tm in (False, True):
        out = gpu_pkg.attention_flash_triton(q, k, v, causal=True, out_token_major=tm)
        torch.cuda.synchronize()
        assert out.shape == ((2, 0, 8, D) if tm else (2, 8, 0, D))


@pytest.mark.parametrize("D", [64, 128])
def test_bf16_v_beyond_f16_range_saturates(gpu_pkg, D):
    """The PV product runs in f16, so bf16 V values beyond the f16 range are
    saturated to +-65504 (the reference keeps bf16's range,
    kernels/attention_kernel.py:221).  Pinned: the output matches the oracle
    over V clamped to +-65504, to 2e-3 plus the f16 rounding of P (2^-11 of
    sum_k w_k |v_k|, with margin) plus one bf16 output rounding, and it is
    measurably different from the unclamped oracle on rows that see a
    saturated key."""
    announce(f"prefill bf16 V beyond the f16 range D={D}")
    q, k, v = qkv(1, 4, 2, 96, 96, D, torch.bfloat16, seed=D)
    v[0, 0, 5, :] = 1.0e5
    v[0, 1, 9, 3] = -3.0e5
    v[0, 0, 70, 7] = 7.0e4
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=True)
    torch.cuda.synchronize()
    qf, kf, vf = f64(q), f64(k), f64(v)
    vc = np.clip(vf, -65504.0, 65504.0)
    ref = O.flash_attention(qf, kf, vc, True)
    mag = O.flash_attention(qf, kf, np.abs(vc), True)            # sum_k w_k |v_k|
    got = f64(out)
    allowed = allowed_error(ref, torch.bfloat16, 2e-3) + 2.0 ** -10 * mag
    err = np.abs(got - ref)
    assert np.isfinite(got).all()
    assert (err <= allowed).all(), f"max err {err.max():.3e} (allowed there {allowed.flat[np.argmax(err - allowed)]:.3e})"
    unclamped = O.flash_attention(qf, kf, vf, True)
    hit = np.abs(unclamped - ref) > 1.0                           # rows/dims a saturated key moves by > 1
    assert hit.any()
    assert (np.abs(got - unclamped)[hit] > 0.5).all()


def test_prefill_errors(gpu_pkg):
    announce("prefill errors")
    q, k, v = qkv(1, 4, 2, 8, 8, 128, torch.bfloat16, seed=1)
    with pytest.raises(AssertionError):
        gpu_pkg.attention_flash_triton(q[..., :48], k[..., :48], v[..., :48], causal=True)
    with pytest.raises(ValueError):
        gpu_pkg.attention_flash_triton(q, k, v.to(torch.float16), causal=True)
