"""Pins for the CPU oracle (``oracle/attention.py``) -- CPU only.

The reference commits no fixtures for this path, so each oracle function is
pinned by checks that do not retype its formula:

* brute-force golden vectors (``tests/golden/*.json``, pure-Python loops);
* a library routine (torch ``scaled_dot_product_attention``, torch rounding);
* closed forms and invariants chosen so that a plausible slip fails one of them
  (kv_len=1 -> v[0]; q=0 -> mean of V; GQA head mapping hq // G rather than
  hq % Hkv; key/page permutation invariance; causal offset; masked rows -> 0;
  split-K merge == unsplit; exact int8 round trip).
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as O
from oracle import eager_path as E

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def _np(x):
    return np.asarray(x, dtype=np.float64)


# --------------------------------------------------------------------- golden


def test_golden_decode():
    g = _load("decode_gqa.json")
    out = O.gqa_decode(_np(g["q"]), _np(g["k"]), _np(g["v"]), g["kv_len"], g["sm_scale"])
    np.testing.assert_allclose(out, _np(g["out"]), rtol=0, atol=1e-12)


@pytest.mark.parametrize("name", ["prefill_causal.json", "prefill_masked.json"])
def test_golden_prefill(name):
    g = _load(name)
    out = O.flash_attention(_np(g["q"]), _np(g["k"]), _np(g["v"]), True, g["sm_scale"])
    np.testing.assert_allclose(out, _np(g["out"]), rtol=0, atol=1e-12)


def test_golden_paged():
    g = _load("paged_decode.json")
    out = O.paged_decode(_np(g["q"]), _np(g["k_pool"]), _np(g["v_pool"]),
                         np.asarray(g["block_table"]), g["kv_len"], g["page_size"], g["sm_scale"])
    np.testing.assert_allclose(out, _np(g["out"]), rtol=0, atol=1e-12)


def test_golden_quant_bit_exact():
    for c in _load("quant_int8.json")["cases"]:
        x = np.asarray(c["x"], dtype=np.float32)
        qi, s = O.quantize_kv_int8(x, "float32", c["scale_dtype"])
        assert qi.tolist() == c["qi"], c
        want = np.float16(c["scale"]) if c["scale_dtype"] == "float16" else np.float32(c["scale"])
        assert s.dtype == want.dtype and s == want, c


def test_golden_splitk():
    g = _load("splitk_merge.json")
    q, k, v = _np(g["q"]), _np(g["k"]), _np(g["v"])
    parts = []
    for p in g["parts"]:
        m, l, acc = O.decode_partial(q, k, v, p["lo"], p["hi"], g["sm_scale"])
        want_m = np.array([-np.inf if x is None else x for x in p["m"]])
        np.testing.assert_allclose(m, want_m, atol=1e-12)
        np.testing.assert_allclose(l, _np(p["l"]), atol=1e-12)
        np.testing.assert_allclose(acc, _np(p["acc"]), atol=1e-12)
        parts.append((m, l, acc))
    np.testing.assert_allclose(O.merge_partials(parts), _np(g["out"]), atol=1e-12)


# ------------------------------------------------------- library cross-checks


def _rand(shape, seed, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * scale


@pytest.mark.parametrize("B,Hq,Hkv,S,D", [(2, 8, 2, 37, 16), (1, 32, 8, 300, 64), (3, 4, 4, 9, 8)])
def test_decode_matches_torch_sdpa(B, Hq, Hkv, S, D):
    q, k, v = _rand((B, Hq, 1, D), 1), _rand((B, Hkv, S, D), 2), _rand((B, Hkv, S, D), 3)
    G = Hq // Hkv
    ref = F.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k).repeat_interleave(G, 1),
        torch.from_numpy(v).repeat_interleave(G, 1)).transpose(1, 2).numpy()
    np.testing.assert_allclose(O.gqa_decode(q, k, v, S), ref, atol=1e-12)


def test_prefill_matches_torch_sdpa_causal():
    B, Hq, Hkv, T, D = 2, 6, 3, 40, 16
    q, k, v = _rand((B, Hq, T, D), 4), _rand((B, Hkv, T, D), 5), _rand((B, Hkv, T, D), 6)
    ref = F.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k).repeat_interleave(2, 1),
        torch.from_numpy(v).repeat_interleave(2, 1), is_causal=True).numpy()
    np.testing.assert_allclose(O.flash_attention(q, k, v, True), ref, atol=1e-12)
    ref_nc = F.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k).repeat_interleave(2, 1),
        torch.from_numpy(v).repeat_interleave(2, 1)).numpy()
    np.testing.assert_allclose(O.flash_attention(q, k, v, False), ref_nc, atol=1e-12)


def test_quant_matches_torch_ops():
    """Bit-exact against torch's own float32 ops on bf16 and fp32 sources."""
    x = torch.randn(64, 8, 128, generator=torch.Generator().manual_seed(7)) * 2.0
    x[0, 0] = 0.0                                 # zero vector (clamp path)
    x[1, 1, :] = 0.0
    x[1, 1, 5] = -1e-3
    for dt, name in ((torch.float32, "float32"), (torch.bfloat16, "bfloat16")):
        xt = x.to(dt)
        amax = xt.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8).float()
        scale = amax / 127.0
        xi = torch.round(xt.float() / scale).clamp_(-127, 127).to(torch.int8)
        for sd in ("float16", "float32"):
            qi, s = O.quantize_kv_int8(xt.float().numpy(), name, sd)
            assert np.array_equal(qi, xi.numpy())
            ts = scale.squeeze(-1).to(torch.float16 if sd == "float16" else torch.float32)
            assert np.array_equal(s, ts.numpy())


def test_eager_path_matches_oracle():
    B, Hq, Hkv, S, D = 2, 8, 2, 50, 32
    q, k, v = _rand((B, Hq, 1, D), 8), _rand((B, Hkv, S, D), 9), _rand((B, Hkv, S, D), 10)
    got = E.eager_gqa(torch.from_numpy(q).float(), torch.from_numpy(k).float(),
                      torch.from_numpy(v).float(), causal=False).numpy()
    np.testing.assert_allclose(got, O.gqa_decode(q, k, v, S), atol=2e-6)


# ------------------------------------------------------ closed forms/invariants


def test_decode_kvlen1_returns_v0():
    q, k, v = _rand((2, 8, 1, 16), 11), _rand((2, 2, 5, 16), 12), _rand((2, 2, 5, 16), 13)
    out = O.gqa_decode(q, k, v, 1)
    for hq in range(8):
        np.testing.assert_array_equal(out[:, 0, hq], v[:, hq // 4, 0])


def test_decode_zero_query_is_mean():
    k, v = _rand((1, 2, 23, 8), 14), _rand((1, 2, 23, 8), 15)
    out = O.gqa_decode(np.zeros((1, 4, 1, 8)), k, v, [17])
    for hq in range(4):
        np.testing.assert_allclose(out[0, 0, hq], v[0, hq // 2, :17].mean(0), atol=1e-13)


def test_decode_gqa_head_mapping():
    """Query head hq must read KV head hq // G (a hq % Hkv slip fails here)."""
    B, Hq, Hkv, S, D = 1, 8, 2, 6, 4
    v = np.zeros((B, Hkv, S, D))
    for h in range(Hkv):
        v[:, h] = h + 1.0
    out = O.gqa_decode(_rand((B, Hq, 1, D), 16), _rand((B, Hkv, S, D), 17), v, S)
    np.testing.assert_allclose(out[0, 0, :, 0], [1, 1, 1, 1, 2, 2, 2, 2], atol=1e-14)


def test_decode_scale_and_sign():
    """Two keys, closed form: o = (v0 + e^{d} v1) / (1 + e^{d}), d = (q.k1 - q.k0) * scale."""
    q = np.array([[[[1.0, 2.0]]]])
    k = np.array([[[[0.5, -1.0], [2.0, 0.25]]]])
    v = np.array([[[[1.0, 0.0], [0.0, 1.0]]]])
    d = ((2.0 + 0.5) - (0.5 - 2.0)) * 0.3
    w = math.exp(d)
    out = O.gqa_decode(q, k, v, 2, sm_scale=0.3)
    np.testing.assert_allclose(out[0, 0, 0], [1 / (1 + w), w / (1 + w)], atol=1e-15)


def test_decode_key_permutation_invariance():
    q, k, v = _rand((1, 4, 1, 8), 18), _rand((1, 1, 30, 8), 19), _rand((1, 1, 30, 8), 20)
    perm = np.random.default_rng(0).permutation(30)
    np.testing.assert_allclose(O.gqa_decode(q, k, v, 30), O.gqa_decode(q, k[:, :, perm], v[:, :, perm], 30),
                               atol=1e-13)


def test_prefill_causal_offset_and_masked_rows():
    B, Hq, Hkv, Tq, Tk, D = 1, 2, 1, 3, 7, 4
    q, k, v = _rand((B, Hq, Tq, D), 21), _rand((B, Hkv, Tk, D), 22), _rand((B, Hkv, Tk, D), 23)
    out = O.flash_attention(q, k, v, True)
    for i in range(Tq):
        n = Tk - Tq + i + 1     # bottom-right: row i sees the first n keys
        want = O.gqa_decode(q[:, :, i:i + 1], k, v, n)[:, 0]
        np.testing.assert_allclose(out[:, :, i], want, atol=1e-13)
    # Tq > Tk: the first Tq - Tk rows see no key at all -> zeros
    q2 = _rand((1, 2, 5, D), 24)
    out2 = O.flash_attention(q2, k[:, :, :2], v[:, :, :2], True)
    np.testing.assert_array_equal(out2[:, :, :3], 0.0)
    assert np.abs(out2[:, :, 3:]).sum() > 0
    # causal row 0 with Tq == Tk is exactly v[0]
    q3 = _rand((1, 2, 7, D), 25)
    np.testing.assert_array_equal(O.flash_attention(q3, k, v, True)[0, :, 0], np.repeat(v[0, :, 0], 2, 0))


def test_paged_identity_and_permutation():
    B, Hq, Hkv, D, page = 3, 4, 2, 8, 4
    lens = np.array([9, 16, 1])
    S = 16
    q, k, v = _rand((B, Hq, 1, D), 26), _rand((B, Hkv, S, D), 27), _rand((B, Hkv, S, D), 28)
    nblk = S // page
    # identity mapping: sequence b owns pages b*nblk .. b*nblk+nblk-1
    k_pool = k.reshape(B, Hkv, nblk, page, D).transpose(0, 2, 1, 3, 4).reshape(B * nblk, Hkv, page, D)
    v_pool = v.reshape(B, Hkv, nblk, page, D).transpose(0, 2, 1, 3, 4).reshape(B * nblk, Hkv, page, D)
    bt = np.arange(B * nblk).reshape(B, nblk)
    ref = O.gqa_decode(q, k, v, lens)
    np.testing.assert_array_equal(O.paged_decode(q, k_pool, v_pool, bt, lens, page), ref)
    perm = np.random.default_rng(1).permutation(B * nblk)
    inv = np.argsort(perm)
    np.testing.assert_array_equal(
        O.paged_decode(q, k_pool[perm], v_pool[perm], inv[bt], lens, page), ref)


def test_int8_exact_roundtrip_matches_float_decode():
    """K/V already on the int8 grid quantise losslessly, so int8 decode == float decode."""
    rng = np.random.default_rng(29)
    B, Hq, Hkv, S, D = 2, 8, 2, 20, 16
    ki = rng.integers(-127, 128, (B, Hkv, S, D))
    ki[..., 0] = 127                           # pin amax so scale is exactly s
    vi = rng.integers(-127, 128, (B, Hkv, S, D))
    vi[..., 0] = -127
    s = np.float32(0.25)
    k = (ki * s).astype(np.float32)
    v = (vi * s).astype(np.float32)
    kq, ks = O.quantize_kv_int8(k, "float32", "float32")
    vq, vs = O.quantize_kv_int8(v, "float32", "float32")
    assert np.array_equal(kq, ki) and np.array_equal(vq, vi)
    q = _rand((B, Hq, 1, D), 30)
    np.testing.assert_allclose(O.int8_decode(q, kq, vq, ks, vs, [20, 7]),
                               O.gqa_decode(q, k, v, [20, 7]), atol=1e-13)


@pytest.mark.parametrize("cuts", [[0, 30], [0, 1, 30], [0, 10, 10, 20, 30], [0, 5, 6, 7, 29, 30]])
def test_splitk_merge_equals_unsplit(cuts):
    q, k, v = _rand((4, 16), 31), _rand((30, 16), 32), _rand((30, 16), 33)
    parts = [O.decode_partial(q, k, v, a, b, 0.25) for a, b in zip(cuts[:-1], cuts[1:])]
    full = O.gqa_decode(q[None, :, None], k[None, None], v[None, None], 30, 0.25)[0, 0]
    np.testing.assert_allclose(O.merge_partials(parts), full, atol=1e-13)
    # associativity: merging a merged pair equals merging all at once
    if len(parts) >= 3:
        m01 = O.merge_partials(parts[:2])
        assert np.isfinite(m01).all()


def test_bf16_rounding_helper():
    x = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, -3.14159, 1e-40], dtype=np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.round_to_bf16(x), want)


# ------------------------------------------------------------- KV write path


def test_paged_write_then_gather_roundtrip():
    """Writing a sequence into permuted pages and gathering it back by the same table is the identity."""
    rng = np.random.default_rng(40)
    B, H, T, D, page = 3, 2, 13, 4, 4
    nblk = 4
    x = rng.standard_normal((B, H, T, D))
    perm = rng.permutation(B * nblk)
    bt = perm.reshape(B, nblk)
    pool = O.kv_write_paged(np.zeros((B * nblk, H, page, D)), x, bt, page, 0)
    for b in range(B):
        np.testing.assert_array_equal(O.paged_gather(pool, bt, b, T, page), x[b])


def test_paged_write_matches_reference_prefill_layout():
    """Sequential tables (allocate()) put token t of b at block b*nblk + t//page, offset t%page:
    the full-block reshape-copy of model/paged_kv_cache.py:97-104, written here with numpy
    reshapes.  (The reference's ragged-tail copy, lines 105-108, transposes (H, tail, D) to
    (tail, H, D) before assigning into (H, tail, D); the layout its docstring states -- token t
    at offset t % page for every head -- is what is pinned here.)"""
    rng = np.random.default_rng(41)
    B, H, T, D, page, nblk = 2, 3, 10, 2, 4, 3
    x = rng.standard_normal((B, H, T, D))
    bt = np.arange(B * nblk).reshape(B, nblk)
    got = O.kv_write_paged(np.zeros((B * nblk, H, page, D)), x, bt, page, 0)
    want = np.zeros((B * nblk, H, page, D))
    full = (T // page) * page
    for b in range(B):
        base = b * nblk
        want[base:base + full // page] = x[b, :, :full].reshape(H, full // page, page, D).transpose(1, 0, 2, 3)
        want[base + full // page, :, :T - full] = x[b, :, full:]
    np.testing.assert_array_equal(got, want)


def test_decode_write_positions_and_bounds():
    """Per-sequence decode positions (seq_lens - 1) land in the right slots; out-of-range ones drop."""
    B, H, D, page = 3, 1, 2, 4
    x = np.arange(B * H * D, dtype=np.float64).reshape(B, H, 1, D) + 1
    bt = np.array([[2, 0], [1, 3], [5, 4]])
    seq_lens = np.array([3, 9, 6])           # token being decoded sits at seq_lens - 1
    pool = O.kv_write_paged(np.zeros((6, H, page, D)), x, bt, page, seq_lens, start_offset=-1)
    np.testing.assert_array_equal(pool[2, :, 2], x[0, :, 0])    # p=2 -> page bt[0][0]=2, slot 2
    np.testing.assert_array_equal(pool[4, :, 1], x[2, :, 0])    # p=5 -> page bt[2][1]=4, slot 1
    # p=8 -> logical block 2, past the 2-block table: dropped
    assert pool.sum() == x[0].sum() + x[2].sum()
    cache = O.kv_write_contiguous(np.zeros((B, H, 5, D)), x, [4, 5, 0])
    np.testing.assert_array_equal(cache[0, :, 4], x[0, :, 0])
    assert not cache[1].any()                                   # position 5 >= S = 5 is dropped
    np.testing.assert_array_equal(cache[2, :, 0], x[2, :, 0])


# ------------------------------------------------- paged INT8-KV GQA decode


def _paged_int8_golden():
    g = _load("paged_int8_decode.json")
    return (_np(g["q"]), np.asarray(g["k_pool"], np.int8), np.asarray(g["v_pool"], np.int8),
            np.asarray(g["k_scale"], np.float32), np.asarray(g["v_scale"], np.float32),
            np.asarray(g["block_table"]), g["kv_len"], g["page_size"], g["sm_scale"], _np(g["out"]))


def test_golden_paged_int8():
    q, kp, vp, ks, vs, bt, lens, page, scale, want = _paged_int8_golden()
    np.testing.assert_allclose(O.paged_int8_decode(q, kp, vp, ks, vs, bt, lens, page, scale), want,
                               rtol=0, atol=1e-12)


def test_golden_paged_int8_detects_scale_slips():
    """The golden vector separates the plausible slips of the scale gather: K and V
    scales swapped, the K scale applied to V as well, and scales read by logical
    (unmapped) page instead of physical page."""
    q, kp, vp, ks, vs, bt, lens, page, scale, want = _paged_int8_golden()
    NB = kp.shape[0]
    logical = np.zeros_like(ks)
    for b in range(bt.shape[0]):
        for j in range(bt.shape[1]):
            logical[bt[b, j]] = ks[j % NB]
    for slip in ((vs, ks), (ks, ks), (logical, vs)):
        got = O.paged_int8_decode(q, kp, vp, slip[0], slip[1], bt, lens, page, scale)
        assert np.abs(got - want).max() > 1e-3


def _paged_int8_case(seed, B=3, Hq=8, Hkv=2, D=16, page=4, lens=(13, 1, 16), nblk=4):
    rng = np.random.default_rng(seed)
    NB = B * nblk
    kp = rng.integers(-127, 128, (NB, Hkv, page, D)).astype(np.int8)
    vp = rng.integers(-127, 128, (NB, Hkv, page, D)).astype(np.int8)
    ks = rng.uniform(0.001, 0.05, (NB, Hkv, page)).astype(np.float32)
    vs = rng.uniform(0.1, 1.0, (NB, Hkv, page)).astype(np.float32)
    q = rng.standard_normal((B, Hq, 1, D)).astype(np.float32)
    return q, kp, vp, ks, vs, np.array(lens), page, nblk


def test_paged_int8_identity_table_equals_contiguous_int8():
    """An identity block table over contiguous caches gives int8_decode bit for bit."""
    q, kp, vp, ks, vs, lens, page, nblk = _paged_int8_case(50)
    B, Hkv, D = q.shape[0], kp.shape[1], kp.shape[3]
    S = nblk * page
    # contiguous (B, Hkv, S, D) view of the same pool: sequence b owns pages b*nblk ...
    k = kp.reshape(B, nblk, Hkv, page, D).transpose(0, 2, 1, 3, 4).reshape(B, Hkv, S, D)
    v = vp.reshape(B, nblk, Hkv, page, D).transpose(0, 2, 1, 3, 4).reshape(B, Hkv, S, D)
    k_s = ks.reshape(B, nblk, Hkv, page).transpose(0, 2, 1, 3).reshape(B, Hkv, S)
    v_s = vs.reshape(B, nblk, Hkv, page).transpose(0, 2, 1, 3).reshape(B, Hkv, S)
    bt = np.arange(B * nblk).reshape(B, nblk)
    np.testing.assert_array_equal(O.paged_int8_decode(q, kp, vp, ks, vs, bt, lens, page),
                                  O.int8_decode(q, k, v, k_s, v_s, lens))


def test_paged_int8_page_permutation_invariance():
    """Moving physical pages (and their scales) and remapping the table changes nothing."""
    q, kp, vp, ks, vs, lens, page, nblk = _paged_int8_case(51)
    bt = np.arange(kp.shape[0]).reshape(q.shape[0], nblk)
    ref = O.paged_int8_decode(q, kp, vp, ks, vs, bt, lens, page)
    perm = np.random.default_rng(52).permutation(kp.shape[0])
    inv = np.argsort(perm)
    got = O.paged_int8_decode(q, kp[perm], vp[perm], ks[perm], vs[perm], inv[bt], lens, page)
    np.testing.assert_array_equal(got, ref)
    # permuting the scales alone (not the pages) must change the result
    bad = O.paged_int8_decode(q, kp, vp, ks[perm], vs[perm], bt, lens, page)
    assert np.abs(bad - ref).max() > 1e-3


def test_eager_paged_int8_matches_oracle():
    """The timed CPU baseline (gather, dequantise, repeat_interleave + SDPA in fp32) agrees
    with the float64 oracle to fp32 rounding: 1e-6 of the output's magnitude (the values
    reach ~100 here, since V scales up to 1.0 times codes up to 127)."""
    q, kp, vp, ks, vs, lens, page, nblk = _paged_int8_case(53)
    perm = np.random.default_rng(54).permutation(kp.shape[0])
    bt = perm.reshape(q.shape[0], nblk).astype(np.int32)
    ref = O.paged_int8_decode(q, kp, vp, ks, vs, bt, lens, page)
    got = E.eager_paged_int8_decode(torch.from_numpy(q), torch.from_numpy(kp), torch.from_numpy(vp),
                                    torch.from_numpy(ks), torch.from_numpy(vs), torch.from_numpy(bt),
                                    torch.from_numpy(lens), page).numpy()
    tol = 1e-6 * np.abs(ref).max()
    np.testing.assert_allclose(got, ref, rtol=0, atol=tol)
    sub = E.eager_paged_int8_decode(torch.from_numpy(q), torch.from_numpy(kp), torch.from_numpy(vp),
                                    torch.from_numpy(ks), torch.from_numpy(vs), torch.from_numpy(bt),
                                    torch.from_numpy(lens), page, batch_rows=[2, 0]).numpy()
    np.testing.assert_allclose(sub, ref[[2, 0]], rtol=0, atol=tol)
