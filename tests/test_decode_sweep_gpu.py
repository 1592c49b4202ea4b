"""Seeded sweep of decode shapes against the float64 oracle.

Each case draws (head_dim, KV heads, GQA group, batch, cache length, layout,
K/V dtype, scale dtype, page size, per-sequence lengths) from a fixed
generator, so a failure names a case that reruns identically.  The shapes
cover how a call's work is cut: odd unit counts (3, 5, 6, 7, 9, 10 KV heads),
groups of more than 16 query heads (two head groups per KV head), single
sequences and batches above and below the CU count (52-127 sequences make
the host halve the units per work-group item to a count that need not divide
the unit count), contiguous caches and paged pools.  Tolerance as in the
other decode tests: 2e-3 before one output rounding, for 16-bit K/V against
the oracle and for int8 against attention over the dequantised cache.
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
N_CASES = 40


def draw(i: int) -> dict:
    r = random.Random(1000 + i)
    while True:
        c = dict(D=r.choice([64, 128, 256]), Hkv=r.choice([1, 2, 3, 4, 5, 6, 7, 8, 9, 10]),
                 G=r.choice([1, 2, 3, 4, 5, 8, 12, 16, 20, 32]),
                 B=r.choice([1, 2, 3, 5, 16, 40, 52, 64, 86, 100, 127, 130]),
                 S=r.choice([16, 100, 700, 2048]), paged=r.random() < 0.5, kv=r.choice(["bf16", "fp16", "int8"]),
                 sd=r.choice([torch.float32, torch.float16]), page=r.choice([16, 32]))
        if c["B"] * c["Hkv"] * c["G"] * c["S"] * c["D"] <= 24_000_000:
            c["lens"] = [r.randint(1, c["S"]) for _ in range(c["B"])]
            if r.random() < 0.3:
                c["lens"] = [c["S"]] * c["B"]
            c["seed"] = 7 + i
            return c


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_decode_shape(gpu_pkg, i):
    c = draw(i)
    announce(f"decode sweep case {i}: {c['kv']} D={c['D']} Hkv={c['Hkv']} G={c['G']} B={c['B']} S={c['S']} "
             f"{'paged p' + str(c['page']) if c['paged'] else 'contiguous'}")
    from importlib import import_module
    syn = import_module("simple-inference-autoresearch_amd.synthetic")
    Hq, Hkv, D = c["Hkv"] * c["G"], c["Hkv"], c["D"]
    qd = torch.float16 if c["kv"] == "fp16" else torch.bfloat16
    int8 = c["kv"] == "int8"
    if c["paged"]:
        case = syn.paged_case(c["lens"], Hq=Hq, Hkv=Hkv, D=D, page=c["page"], seed=c["seed"], device=DEV,
                              kv=c["kv"], q_dtype=qd, scale_dtype=c["sd"])
        if int8:
            out = gpu_pkg.paged_gqa_int8_flash_decode(case.q, case.k_pool, case.v_pool, case.k_scale, case.v_scale,
                                                      case.block_table, case.kv_len, case.page_size)
            ref = O.paged_int8_decode(f64(case.q), case.k_pool.cpu().numpy(), case.v_pool.cpu().numpy(),
                                      f64(case.k_scale), f64(case.v_scale), case.block_table.cpu().numpy(),
                                      case.ctx, case.page_size)
        else:
            out = gpu_pkg.paged_attention_flash_decode(case.q, case.k_pool, case.v_pool, case.block_table,
                                                       case.kv_len, case.page_size)
            ref = O.paged_decode(f64(case.q), f64(case.k_pool), f64(case.v_pool), case.block_table.cpu().numpy(),
                                 case.ctx, case.page_size)
    else:
        g = torch.Generator(device=DEV).manual_seed(c["seed"])
        B, S = c["B"], c["S"]
        q = torch.randn(B, Hq, 1, D, generator=g, device=DEV).to(qd)
        k = torch.randn(B, Hkv, S, D, generator=g, device=DEV)
        v = torch.randn(B, Hkv, S, D, generator=g, device=DEV)
        kl = torch.tensor(c["lens"], dtype=torch.int32, device=DEV)
        if int8:
            ki, ks = syn.quantize_per_vector(k, c["sd"])
            vi, vs = syn.quantize_per_vector(v, c["sd"])
            out = gpu_pkg.gqa_int8_flash_decode(q, ki, vi, ks, vs, kl)
            ref = O.int8_decode(f64(q), ki.cpu().numpy(), vi.cpu().numpy(), f64(ks), f64(vs), c["lens"])
        else:
            kd = torch.float16 if c["kv"] == "fp16" else torch.bfloat16
            k, v = k.to(kd), v.to(kd)
            out = gpu_pkg.attention_flash_decode(q, k, v, kl)
            ref = O.gqa_decode(f64(q), f64(k), f64(v), c["lens"])
    torch.cuda.synchronize()
    assert_close(out, ref, 2e-3, f"case {i} {c}")
