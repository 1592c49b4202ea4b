"""Seeded sweep of prefill shapes against the float64 oracle.

Each case draws (head_dim, KV heads, GQA group, batch, query and key lengths,
causal, dtype, output layout) from a fixed generator, so a failure names a
case that reruns identically.  The draws span both work-group variants at
head_dim 128 (grids below and above the CU count), chunked prefill (Tq < Tk)
and Tq > Tk (leading rows see no key), one and several head groups per KV
head.  A second sweep draws float16 shapes at head_dim 32-128, whose V is
read in place, with q, k and v stored contiguously, token-major or as row
slices of a wider buffer.  Tolerance as in the other prefill tests: 2e-3
before one rounding to the output dtype.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from helpers import announce, assert_close, f64
from oracle import attention as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
N_CASES = 24


def draw(i: int) -> dict:
    r = random.Random(5000 + i)
    while True:
        Tk = r.choice([1, 40, 64, 129, 300, 700, 1100])
        shape = r.random()
        Tq = Tk if shape < 0.5 else (r.randint(1, Tk) if shape < 0.8 else Tk + r.randint(1, 80))
        c = dict(D=r.choice([16, 32, 64, 128, 128, 256]), Hkv=r.choice([1, 2, 4, 8]), G=r.choice([1, 2, 3, 4, 8]),
                 B=r.choice([1, 2, 4]), Tq=Tq, Tk=Tk, causal=r.random() < 0.7,
                 dtype=r.choice([torch.bfloat16, torch.float16]), token_major=r.random() < 0.3, seed=31 + i)
        if c["B"] * c["Hkv"] * c["G"] * c["Tq"] * c["Tk"] * c["D"] <= 400_000_000:
            return c


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_prefill_shape(gpu_pkg, i):
    c = draw(i)
    announce(f"prefill sweep case {i}: D={c['D']} Hkv={c['Hkv']} G={c['G']} B={c['B']} Tq={c['Tq']} Tk={c['Tk']} "
             f"causal={c['causal']} {c['dtype']}")
    B, Hkv, D = c["B"], c["Hkv"], c["D"]
    Hq = Hkv * c["G"]
    g = torch.Generator(device=DEV).manual_seed(c["seed"])
    q = (torch.randn(B, Hq, c["Tq"], D, generator=g, device=DEV) * 0.5).to(c["dtype"])
    k = (torch.randn(B, Hkv, c["Tk"], D, generator=g, device=DEV) * 0.5).to(c["dtype"])
    v = (torch.randn(B, Hkv, c["Tk"], D, generator=g, device=DEV) * 0.5).to(c["dtype"])
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=c["causal"], out_token_major=c["token_major"])
    torch.cuda.synchronize()
    if c["token_major"]:
        out = out.transpose(1, 2)
    ref = O.flash_attention(f64(q), f64(k), f64(v), c["causal"])
    assert_close(out, ref, 2e-3, f"case {i} {c}")


def draw_f16(i: int) -> dict:
    r = random.Random(7000 + i)
    while True:
        Tk = r.choice([1, 33, 64, 65, 250, 513, 1000, 1500])
        shape = r.random()
        Tq = Tk if shape < 0.5 else (r.randint(1, Tk) if shape < 0.8 else Tk + r.randint(1, 80))
        c = dict(D=r.choice([32, 64, 128, 128]), Hkv=r.choice([1, 2, 4, 8]), G=r.choice([1, 2, 4, 8]),
                 B=r.choice([1, 2, 3]), Tq=Tq, Tk=Tk, causal=r.random() < 0.7,
                 layout=r.choice(["contiguous", "token_major", "padded_rows"]), seed=91 + i)
        if c["B"] * c["Hkv"] * c["G"] * c["Tq"] * c["Tk"] * c["D"] <= 400_000_000:
            return c


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_f16_in_place_v(gpu_pkg, i):
    """float16 at head_dim 32-128 reads V in place (raw rows, transposed LDS
    reads): seeded shapes with V (and q, k) as contiguous tensors, as
    token-major (B, T, H, D) storage, or as row slices of a wider buffer
    (rows (D + 32) elements apart), every element against the oracle."""
    c = draw_f16(i)
    announce(f"prefill f16 in-place V case {i}: {c}")
    B, Hkv, D = c["B"], c["Hkv"], c["D"]
    Hq = Hkv * c["G"]
    g = torch.Generator(device=DEV).manual_seed(c["seed"])

    def make(H, T):
        if c["layout"] == "token_major":
            return (torch.randn(B, T, H, D, generator=g, device=DEV) * 0.5).half().transpose(1, 2)
        if c["layout"] == "padded_rows":
            return (torch.randn(B, H, T, D + 32, generator=g, device=DEV) * 0.5).half()[..., :D]
        return (torch.randn(B, H, T, D, generator=g, device=DEV) * 0.5).half()

    q, k, v = make(Hq, c["Tq"]), make(Hkv, c["Tk"]), make(Hkv, c["Tk"])
    out = gpu_pkg.attention_flash_triton(q, k, v, causal=c["causal"])
    torch.cuda.synchronize()
    ref = O.flash_attention(f64(q), f64(k), f64(v), c["causal"])
    assert_close(out, ref, 2e-3, f"case {i} {c}")
