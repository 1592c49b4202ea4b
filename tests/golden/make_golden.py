"""Write the golden vectors in this folder by brute force.

Run:  python tests/golden/make_golden.py

The reference repository commits no fixtures or known-answer tests for its
attention path, so these vectors pin the numpy oracle (``oracle/attention.py``)
from the mathematics instead: every expected output below is computed with
plain Python loops, ``math.exp`` and an explicit float32 emulation, written
independently of the oracle's vectorised code.  Inputs come from a fixed
32-bit LCG so the file is reproducible without numpy's RNG.

Cases
-----
decode_gqa.json      single-query GQA decode, per-sequence kv_len (incl. 1 and S)
prefill_causal.json  causal attention with Tq < Tk (bottom-right offset)
prefill_masked.json  causal with Tq > Tk: leading rows fully masked -> zeros
paged_decode.json    paged pool with a permuted block table, ragged lengths
paged_int8_decode.json  paged int8 pools with distinct per-token-per-head K and V
                     scale pools, GQA, a permuted block table, ragged lengths
quant_int8.json      per-vector int8 quantisation known answers
splitk_merge.json    (m, l, acc) partials over key ranges and their merge
"""

from __future__ import annotations

import json
import math
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))


class LCG:
    """Numerical Recipes LCG; values uniform in [-1, 1) with 24-bit resolution."""

    def __init__(self, seed: int):
        self.x = seed & 0xFFFFFFFF

    def next(self) -> float:
        self.x = (1664525 * self.x + 1013904223) & 0xFFFFFFFF
        return ((self.x >> 8) / float(1 << 24)) * 2.0 - 1.0

    def tensor(self, shape, scale=1.0):
        if len(shape) == 1:
            return [self.next() * scale for _ in range(shape[0])]
        return [self.tensor(shape[1:], scale) for _ in range(shape[0])]


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def f16(x: float) -> float:
    return struct.unpack("<e", struct.pack("<e", x))[0]


def softmax_rows(q, keys, vals, scale):
    """q: list[D]; keys/vals: list of list[D]. Returns list[D]."""
    if not keys:
        return [0.0] * len(q)
    s = [sum(qi * ki for qi, ki in zip(q, k)) * scale for k in keys]
    m = max(s)
    e = [math.exp(x - m) for x in s]
    tot = sum(e)
    return [sum(e[n] * vals[n][d] for n in range(len(vals))) / tot for d in range(len(q))]


def case_decode():
    r = LCG(11)
    B, Hq, Hkv, S, D = 3, 4, 2, 5, 4
    q = r.tensor([B, Hq, 1, D])
    k = r.tensor([B, Hkv, S, D])
    v = r.tensor([B, Hkv, S, D])
    kv_len = [3, 5, 1]
    scale = 0.7
    G = Hq // Hkv
    out = [[[None] * Hq] for _ in range(B)]
    for b in range(B):
        for hq in range(Hq):
            h = hq // G
            n = kv_len[b]
            out[b][0][hq] = softmax_rows(q[b][hq][0], k[b][h][:n], v[b][h][:n], scale)
    return dict(q=q, k=k, v=v, kv_len=kv_len, sm_scale=scale, out=out)


def causal_attention(q, k, v, scale):
    """q: (B,Hq,Tq,D) nested lists; bottom-right causal; masked rows -> 0."""
    B, Hq, Tq = len(q), len(q[0]), len(q[0][0])
    Hkv, Tk = len(k[0]), len(k[0][0])
    G = Hq // Hkv
    out = []
    for b in range(B):
        ob = []
        for hq in range(Hq):
            h = hq // G
            oh = []
            for i in range(Tq):
                last = (Tk - Tq) + i
                keys = [k[b][h][j] for j in range(Tk) if j <= last]
                vals = [v[b][h][j] for j in range(Tk) if j <= last]
                oh.append(softmax_rows(q[b][hq][i], keys, vals, scale))
            ob.append(oh)
        out.append(ob)
    return out


def case_prefill(seed, B, Hq, Hkv, Tq, Tk, D, scale):
    r = LCG(seed)
    q = r.tensor([B, Hq, Tq, D])
    k = r.tensor([B, Hkv, Tk, D])
    v = r.tensor([B, Hkv, Tk, D])
    return dict(q=q, k=k, v=v, causal=True, sm_scale=scale, out=causal_attention(q, k, v, scale))


def case_paged():
    r = LCG(29)
    B, Hq, Hkv, D, page = 2, 2, 1, 3, 2
    kv_len = [5, 3]
    nblk = [3, 2]
    NB = 6
    k_pool = r.tensor([NB, Hkv, page, D])
    v_pool = r.tensor([NB, Hkv, page, D])
    block_table = [[4, 0, 5], [2, 1, 0]]          # row 1's third entry is unused padding
    scale = 0.9
    q = r.tensor([B, Hq, 1, D])
    out = []
    for b in range(B):
        keys = [k_pool[block_table[b][t // page]][0][t % page] for t in range(kv_len[b])]
        vals = [v_pool[block_table[b][t // page]][0][t % page] for t in range(kv_len[b])]
        out.append([[softmax_rows(q[b][hq][0], keys, vals, scale) for hq in range(Hq)]])
    return dict(q=q, k_pool=k_pool, v_pool=v_pool, block_table=block_table, kv_len=kv_len,
                page_size=page, sm_scale=scale, nblk=nblk, out=out)


def case_paged_int8():
    """Paged INT8-KV GQA decode by hand: token t of sequence b is slot t % page of
    page block_table[b][t // page]; its key is k_i8 * k_scale and its value
    v_i8 * v_scale, both scales read at (page, kv head, slot).  K and V scales
    are drawn from different ranges, so swapping them changes the output."""
    r = LCG(53)
    B, Hq, Hkv, D, page = 2, 4, 2, 3, 2
    NB = 7
    kv_len = [5, 4]
    block_table = [[6, 1, 3], [0, 4, 2]]          # row 1's third entry is unused padding

    def i8_tensor(shape):
        if len(shape) == 1:
            return [int(round(r.next() * 127.0)) for _ in range(shape[0])]
        return [i8_tensor(shape[1:]) for _ in range(shape[0])]

    def f32_tensor(shape, lo, hi):
        if len(shape) == 1:
            return [f32(lo + (hi - lo) * (r.next() + 1.0) / 2.0) for _ in range(shape[0])]
        return [f32_tensor(shape[1:], lo, hi) for _ in range(shape[0])]

    k_pool = i8_tensor([NB, Hkv, page, D])
    v_pool = i8_tensor([NB, Hkv, page, D])
    k_scale = f32_tensor([NB, Hkv, page], 0.002, 0.02)
    v_scale = f32_tensor([NB, Hkv, page], 0.05, 0.5)
    q = r.tensor([B, Hq, 1, D], 3.0)
    scale = 0.6
    G = Hq // Hkv
    out = []
    for b in range(B):
        rows = []
        for hq in range(Hq):
            h = hq // G
            keys, vals = [], []
            for t in range(kv_len[b]):
                pg, slot = block_table[b][t // page], t % page
                keys.append([k_pool[pg][h][slot][d] * k_scale[pg][h][slot] for d in range(D)])
                vals.append([v_pool[pg][h][slot][d] * v_scale[pg][h][slot] for d in range(D)])
            rows.append(softmax_rows(q[b][hq][0], keys, vals, scale))
        out.append([rows])
    return dict(q=q, k_pool=k_pool, v_pool=v_pool, k_scale=k_scale, v_scale=v_scale,
                block_table=block_table, kv_len=kv_len, page_size=page, sm_scale=scale, out=out)


def quant_vec(x, scale_dtype):
    """model/kv_cache.py:58-67 by hand, float32 emulated with struct."""
    xs = [f32(e) for e in x]
    amax = max(abs(e) for e in xs)
    amax = max(amax, f32(1e-8))
    scale = f32(amax / 127.0)
    qi = []
    for e in xs:
        t = f32(e / scale)
        rq = round(t)                      # Python round() is half-to-even
        qi.append(max(-127, min(127, int(rq))))
    s_out = f16(scale) if scale_dtype == "float16" else scale
    return qi, s_out


def case_quant():
    vectors = [
        [0.0, 0.0, 0.0, 0.0],                       # zero vector: scale = 1e-8/127, all zeros
        [127.0, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, -1.5],  # scale exactly 1: ties go to even
        [-3.0, 0.0, 0.0, 0.0],                      # one-hot: -> -127
        [1.0, 2.0, 3.0, 4.0],
        [0.001, -0.002, 0.0005, 0.0],
    ]
    r = LCG(5)
    vectors.append([r.next() * 3.0 for _ in range(16)])
    out = []
    for x in vectors:
        for sd in ("float32", "float16"):
            qi, s = quant_vec(x, sd)
            out.append(dict(x=x, scale_dtype=sd, qi=qi, scale=s))
    return dict(cases=out)


def case_splitk():
    r = LCG(41)
    G, n, D = 2, 7, 3
    q = r.tensor([G, D])
    k = r.tensor([n, D])
    v = r.tensor([n, D])
    scale = 1.3
    bounds = [(0, 3), (3, 3), (3, 7)]                 # includes an empty split
    parts = []
    for lo, hi in bounds:
        ms, ls, accs = [], [], []
        for g in range(G):
            if hi <= lo:
                ms.append(None)
                ls.append(0.0)
                accs.append([0.0] * D)
                continue
            s = [sum(q[g][d] * k[j][d] for d in range(D)) * scale for j in range(lo, hi)]
            m = max(s)
            e = [math.exp(x - m) for x in s]
            ms.append(m)
            ls.append(sum(e))
            accs.append([sum(e[t] * v[lo + t][d] for t in range(hi - lo)) for d in range(D)])
        parts.append(dict(lo=lo, hi=hi, m=ms, l=ls, acc=accs))
    full = [softmax_rows(q[g], k, v, scale) for g in range(G)]
    return dict(q=q, k=k, v=v, sm_scale=scale, parts=parts, out=full)


def main():
    cases = {
        "decode_gqa.json": case_decode(),
        "prefill_causal.json": case_prefill(17, 1, 4, 2, 3, 6, 3, 0.8),
        "prefill_masked.json": case_prefill(23, 1, 2, 1, 4, 2, 3, 1.1),
        "paged_decode.json": case_paged(),
        "paged_int8_decode.json": case_paged_int8(),
        "quant_int8.json": case_quant(),
        "splitk_merge.json": case_splitk(),
    }
    for name, data in cases.items():
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(data, f, indent=None, separators=(",", ":"))
        print("wrote", name)


if __name__ == "__main__":
    main()
