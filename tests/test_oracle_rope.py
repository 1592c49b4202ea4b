"""CPU pins of the RoPE oracle and the host side of the RoPE drop-in.

``oracle.rope.rope_qk`` restates ``kernels/rope_kernel.py:86-165``.  It is
pinned here by checks that do not retype its formula:

* transformers' Llama ``apply_rotary_pos_emb`` (split-half, ``x*cos +
  rotate_half(x)*sin``) and GPT-J ``apply_rotary_pos_emb`` (adjacent pairs,
  ``rotate_every_two``), both evaluated by torch in float32 on the CPU with
  every operation rounded separately: equal bit for bit (a swapped pair, a
  wrong sign or a transposed table fails);
* complex128 multiplication ``(x_a + i x_b)(cos + i sin)``: within the fp32
  rounding of two products and a sum;
* position 0 (cos 1, sin 0) returns the input unchanged, in every dtype;
* rotation by a true angle keeps each pair's norm;
* duplicated ``(T, D)`` and raw ``(T, D/2)`` tables give identical output,
  and row ``r`` uses table row ``r % Tc`` (decode tables of one row, and
  batch rows sharing a prefill table).

The host-side checks of the drop-in (table validation errors, llama3
frequency scaling against transformers) need no GPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import rope as OR

RNG = np.random.default_rng(1234)


def randn(*shape, dtype="float32"):
    return OA.round_to_dtype(RNG.standard_normal(shape).astype(np.float32), dtype)


def angles(T, D, theta=10000.0, start=0):
    inv = 1.0 / theta ** (np.arange(0, D, 2, dtype=np.float64) / D)
    return np.outer(np.arange(start, start + T, dtype=np.float64), inv)


def tables(T, D, dtype="float32", duplicated=True, start=0):
    a = angles(T, D, start=start)
    c, s = np.cos(a), np.sin(a)
    if duplicated:
        c, s = np.concatenate([c, c], -1), np.concatenate([s, s], -1)
    return OA.round_to_dtype(c.astype(np.float32), dtype), OA.round_to_dtype(s.astype(np.float32), dtype)


@pytest.mark.parametrize("D", [8, 64, 128])
def test_split_half_equals_transformers_llama(D):
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    B, T, Hq, Hkv = 2, 5, 4, 2
    q, k = randn(B, T, Hq, D), randn(B, T, Hkv, D)
    c, s = tables(T, D)
    cq, sq = torch.from_numpy(c).expand(B, T, D), torch.from_numpy(s).expand(B, T, D)
    rq, rk = apply_rotary_pos_emb(torch.from_numpy(q), torch.from_numpy(k), cq, sq, unsqueeze_dim=2)
    oq, ok = OR.rope_qk(q, k, c, s)
    assert np.array_equal(oq, rq.numpy()) and np.array_equal(ok, rk.numpy())


@pytest.mark.parametrize("D", [8, 64, 128])
def test_interleaved_equals_transformers_gptj(D):
    from transformers.models.gptj.modeling_gptj import apply_rotary_pos_emb

    B, T, Hq, Hkv = 2, 5, 4, 2
    q, k = randn(B, T, Hq, D), randn(B, T, Hkv, D)
    c, s = tables(T, D, duplicated=False)
    cg = torch.from_numpy(c).expand(B, T, D // 2)
    sg = torch.from_numpy(s).expand(B, T, D // 2)
    rq = apply_rotary_pos_emb(torch.from_numpy(q), sg, cg)
    rk = apply_rotary_pos_emb(torch.from_numpy(k), sg, cg)
    oq, ok = OR.rope_qk(q, k, c, s, interleaved=True)
    assert np.array_equal(oq, rq.numpy()) and np.array_equal(ok, rk.numpy())


@pytest.mark.parametrize("interleaved", [False, True])
def test_complex_multiplication(interleaved):
    B, T, H, D = 3, 7, 2, 32
    x = randn(B, T, H, D)
    c, s = tables(T, D, duplicated=False)
    got, _ = OR.rope_qk(x, x[:, :, :1], c, s, interleaved=interleaved)
    x64 = x.astype(np.float64)
    if interleaved:
        z = x64[..., 0::2] + 1j * x64[..., 1::2]
    else:
        z = x64[..., : D // 2] + 1j * x64[..., D // 2:]
    w = (c.astype(np.float64) + 1j * s.astype(np.float64))[None, :, None, :]
    r = z * w
    ga, gb = (got[..., 0::2], got[..., 1::2]) if interleaved else (got[..., : D // 2], got[..., D // 2:])
    bound = 2.0 ** -22 * (np.abs(z.real * w.real) + np.abs(z.imag * w.imag) + np.abs(z.imag * w.real)
                          + np.abs(z.real * w.imag)) + 1e-30
    assert (np.abs(ga - r.real) <= bound).all()
    assert (np.abs(gb - r.imag) <= bound).all()


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("interleaved", [False, True])
def test_position_zero_is_identity(dtype, interleaved):
    q, k = randn(2, 3, 4, 64, dtype=dtype), randn(2, 3, 1, 64, dtype=dtype)
    c, s = tables(1, 64, dtype=dtype)
    oq, ok = OR.rope_qk(q, k, c, s, interleaved=interleaved, dtype=dtype)
    assert np.array_equal(oq, q) and np.array_equal(ok, k)


def test_pair_norm_preserved():
    D = 128
    x = randn(1, 16, 2, D)
    c, s = tables(16, D, start=1000)
    got, _ = OR.rope_qk(x, x, c, s)
    n_in = x[..., : D // 2].astype(np.float64) ** 2 + x[..., D // 2:].astype(np.float64) ** 2
    n_out = got[..., : D // 2].astype(np.float64) ** 2 + got[..., D // 2:].astype(np.float64) ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=2e-6, atol=1e-12)


def test_duplicated_and_raw_tables_agree():
    q, k = randn(2, 6, 3, 96), randn(2, 6, 1, 96)
    cd, sd = tables(6, 96)
    cr, sr = tables(6, 96, duplicated=False)
    for il in (False, True):
        a = OR.rope_qk(q, k, cd, sd, interleaved=il)
        b = OR.rope_qk(q, k, cr, sr, interleaved=il)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_table_row_is_row_mod_rows():
    # decode: a one-row table serves every batch row
    q, k = randn(5, 1, 2, 32), randn(5, 1, 1, 32)
    c, s = tables(1, 32, start=77)
    whole = OR.rope_qk(q, k, c, s)
    for b in range(5):
        one = OR.rope_qk(q[b:b + 1], k[b:b + 1], c, s)
        assert np.array_equal(whole[0][b:b + 1], one[0]) and np.array_equal(whole[1][b:b + 1], one[1])
    # prefill: every sequence of the batch starts at table row 0
    q, k = randn(3, 4, 2, 32), randn(3, 4, 1, 32)
    c, s = tables(4, 32)
    whole = OR.rope_qk(q, k, c, s)
    for b in range(3):
        one = OR.rope_qk(q[b:b + 1], k[b:b + 1], c, s)
        assert np.array_equal(whole[0][b:b + 1], one[0])


def test_planted_sign_error_is_caught():
    """A sign slip in the restatement fails the transformers pin."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    q = randn(1, 3, 2, 16)
    c, s = tables(3, 16)
    rq, _ = apply_rotary_pos_emb(torch.from_numpy(q), torch.from_numpy(q), torch.from_numpy(c)[None],
                                 torch.from_numpy(s)[None], unsqueeze_dim=2)
    oq, _ = OR.rope_qk(q, q, c, -s)
    assert not np.array_equal(oq, rq.numpy())


# ------------------------------------------------------------ host side of the drop-in


def test_llama3_frequencies_match_transformers(pkg):
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import _compute_llama3_parameters

    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, head_dim=128, max_position_embeddings=131072,
                      rope_parameters={"rope_type": "llama3", "rope_theta": 500000.0, "factor": 32.0,
                                       "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                       "original_max_position_embeddings": 8192})
    inv, _ = _compute_llama3_parameters(cfg, "cpu")
    rf = pkg.RopeFrequencies(128, 32, device=torch.device("cpu"))
    base = 1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    mine = rf._llama3_scaled(base, 32.0, 1.0, 4.0, 8192)
    torch.testing.assert_close(mine, inv, rtol=1e-6, atol=0)
    ang = torch.outer(torch.arange(32, dtype=torch.float32), mine)
    assert torch.equal(rf.cos, torch.cat([ang, ang], -1).cos())
    c16, s16 = rf.get(4, start_pos=3, dtype=torch.bfloat16)
    assert torch.equal(c16, rf.cos.to(torch.bfloat16)[3:7]) and torch.equal(s16, rf.sin.to(torch.bfloat16)[3:7])


def test_table_validation_errors(pkg):
    q = torch.zeros(1, 2, 2, 8)
    k = torch.zeros(1, 2, 1, 8)
    with pytest.raises(ValueError, match="head_dim"):
        pkg.rope_triton(q, k, torch.zeros(2, 6), torch.zeros(2, 6))
    with pytest.raises(ValueError, match="identical shape"):
        pkg.rope_triton(q, k, torch.zeros(2, 8), torch.zeros(3, 8))
    with pytest.raises(ValueError, match="unit-stride"):
        pkg.rope_triton(q, k, torch.zeros(8, 2).t(), torch.zeros(8, 2).t())
    with pytest.raises(ValueError, match="row stride"):
        pkg.rope_triton(q, k, torch.zeros(2, 8), torch.zeros(2, 16)[:, :8])
