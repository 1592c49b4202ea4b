"""Decode geometries whose units per work-group item do not divide the unit count.

The host picks the units per item (IU) of a decode call: min(U, waves) halved
while the batch has fewer items than CUs.  IU need not divide U (U = KV heads
x head groups): with 10 KV heads, 4 query heads each, D = 128 and 100
sequences it is 4 (three unit blocks, the last holding 2 of its 4 slots) with
two waves per unit; with 5 KV heads at D = 256 (4-wave work-groups) it is 2.
The two waves of a unit merge through LDS, and the slots past the last unit
own no output row.  Every output row is compared with the float64 oracle
(2e-3 before one output rounding; int8 against the dequantised cache at
1e-2), for contiguous caches and paged pools, with short equal lengths (every
segment written directly) and longer ragged ones (split-K pieces).  A call
through the C ABI writes into a view of a larger buffer whose rows before and
after hold a sentinel that must survive.  A last test covers calls with one
shared length whose segments are a multiple of the persistent grid: those
run the main kernel alone, which then also writes the zero rows of a zero
length.
"""

from __future__ import annotations

import ctypes
import importlib

import pytest
import torch

from helpers import announce, assert_close, f64
from oracle import attention as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
syn = importlib.import_module("simple-inference-autoresearch_amd.synthetic")
L = importlib.import_module("simple-inference-autoresearch_amd._lib")

SHAPES = [(128, 10, 4, 100), (256, 5, 4, 100), (128, 9, 4, 60), (128, 7, 20, 90)]


def lengths(B: int, kind: str):
    if kind == "short":
        return [40] * B
    g = torch.Generator().manual_seed(B)
    return torch.randint(1, 900, (B,), generator=g).tolist()


@pytest.mark.parametrize("kind", ["short", "ragged"])
@pytest.mark.parametrize("D,Hkv,G,B", SHAPES)
def test_contiguous(gpu_pkg, D, Hkv, G, B, kind):
    announce(f"item-width decode contiguous D={D} Hkv={Hkv} G={G} B={B} {kind}")
    Hq = Hkv * G
    lens = lengths(B, kind)
    S = max(lens)
    g = torch.Generator(device=DEV).manual_seed(D + Hkv + B)
    q = torch.randn(B, Hq, 1, D, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g, device=DEV)
    v = torch.randn(B, Hkv, S, D, generator=g, device=DEV)
    kl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = gpu_pkg.attention_flash_decode(q, k.to(torch.bfloat16), v.to(torch.bfloat16), kl)
    torch.cuda.synchronize()
    ref = O.gqa_decode(f64(q), f64(k.to(torch.bfloat16)), f64(v.to(torch.bfloat16)), lens)
    assert_close(out, ref, 2e-3, "bf16")
    ki, ks = syn.quantize_per_vector(k, torch.float32)
    vi, vs = syn.quantize_per_vector(v, torch.float32)
    out8 = gpu_pkg.gqa_int8_flash_decode(q, ki, vi, ks, vs, kl)
    torch.cuda.synchronize()
    ref8 = O.int8_decode(f64(q), ki.cpu().numpy(), vi.cpu().numpy(), f64(ks), f64(vs), lens)
    assert_close(out8, ref8, 1e-2, "int8")


@pytest.mark.parametrize("kind", ["short", "ragged"])
@pytest.mark.parametrize("D,Hkv,G,B", SHAPES)
def test_paged(gpu_pkg, D, Hkv, G, B, kind):
    announce(f"item-width decode paged D={D} Hkv={Hkv} G={G} B={B} {kind}")
    Hq = Hkv * G
    lens = lengths(B, kind)
    case = syn.paged_case(lens, Hq=Hq, Hkv=Hkv, D=D, page=16, seed=B + D, device=DEV, kv="bf16",
                          q_dtype=torch.bfloat16)
    out = gpu_pkg.paged_attention_flash_decode(case.q, case.k_pool, case.v_pool, case.block_table, case.kv_len,
                                               case.page_size)
    torch.cuda.synchronize()
    ref = O.paged_decode(f64(case.q), f64(case.k_pool), f64(case.v_pool), case.block_table.cpu().numpy(),
                         case.ctx, case.page_size)
    assert_close(out, ref, 2e-3, "paged bf16")
    c8 = syn.paged_case(lens, Hq=Hq, Hkv=Hkv, D=D, page=16, seed=B + D + 1, device=DEV, kv="int8")
    out8 = gpu_pkg.paged_gqa_int8_flash_decode(c8.q, c8.k_pool, c8.v_pool, c8.k_scale, c8.v_scale, c8.block_table,
                                               c8.kv_len, c8.page_size)
    torch.cuda.synchronize()
    ref8 = O.paged_int8_decode(f64(c8.q), c8.k_pool.cpu().numpy(), c8.v_pool.cpu().numpy(), f64(c8.k_scale),
                               f64(c8.v_scale), c8.block_table.cpu().numpy(), c8.ctx, c8.page_size)
    assert_close(out8, ref8, 1e-2, "paged int8")


@pytest.mark.parametrize("D,Hkv,G,B", SHAPES[:2])
def test_capi_output_guard(gpu_pkg, D, Hkv, G, B):
    """The output is a view of rows 1..B of a (B + 2)-row buffer: rows 0 and
    B + 1 keep their sentinel bits, and rows 1..B match the oracle."""
    h = L.require_library()
    announce(f"item-width decode C ABI output guard D={D} Hkv={Hkv} G={G} B={B}")
    Hq = Hkv * G
    lens = [40] * B
    case = syn.paged_case(lens, Hq=Hq, Hkv=Hkv, D=D, page=16, seed=5 + D, device=DEV, kv="bf16",
                          q_dtype=torch.bfloat16)
    sentinel = 0x7F81   # a bf16 NaN pattern no kernel writes
    buf = torch.full((B + 2, 1, Hq, D), sentinel, dtype=torch.int16, device=DEV)
    out = buf[1:B + 1].view(torch.bfloat16)
    ws = torch.empty(gpu_pkg.decode_workspace_size(B, Hq, Hkv, D), dtype=torch.uint8, device=DEV)
    ds = [L.desc(t) for t in (case.q, case.k_pool, case.v_pool, case.block_table, case.kv_len)]
    do = L.desc(out)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = h.sia_paged_attention_flash_decode(*[ctypes.byref(d) for d in ds], ctypes.c_int32(16),
                                            ctypes.c_float(D ** -0.5), ctypes.byref(do),
                                            ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(ws.numel()), None,
                                            stream)
    assert rc == 0, h.sia_last_error_message()
    torch.cuda.synchronize()
    assert bool((buf[0] == sentinel).all()), "row before the output was written"
    assert bool((buf[B + 1] == sentinel).all()), "row after the output was written"
    ref = O.paged_decode(f64(case.q), f64(case.k_pool), f64(case.v_pool), case.block_table.cpu().numpy(),
                         case.ctx, case.page_size)
    assert_close(out, ref, 2e-3, "C ABI paged bf16")


@pytest.mark.parametrize("kv", ["bf16", "int8"])
@pytest.mark.parametrize("paged", [False, True])
def test_shared_length_whole_segment_split(gpu_pkg, kv, paged):
    """One shared length (kv_len of one element) over 64 sequences x 8 KV heads:
    the segments are a multiple of the persistent grid, every group gets whole
    segments and the call is the main kernel alone (no merge kernel).  Lengths
    0 (every row zero), 1, 100 and 1000, through the C ABI into a NaN-filled
    output, against the float64 oracle."""
    h = L.require_library()
    B, Hq, Hkv, D = 64, 32, 8, 128
    for n in (0, 1, 100, 1000):
        announce(f"shared length {n}: {kv} {'paged' if paged else 'contiguous'} B={B}")
        if paged:
            case = syn.paged_case([max(n, 1)] * B, Hq=Hq, Hkv=Hkv, D=D, page=16, seed=7 + n, device=DEV, kv=kv,
                                  q_dtype=torch.bfloat16, per_seq_len=False)
            tensors = [case.q, case.k_pool, case.v_pool] + ([case.k_scale, case.v_scale] if kv == "int8" else []) + \
                      [case.block_table]
            q = case.q
        else:
            g = torch.Generator(device=DEV).manual_seed(n)
            q = torch.randn(B, Hq, 1, D, generator=g, device=DEV).to(torch.bfloat16)
            kf = torch.randn(B, Hkv, max(n, 1), D, generator=g, device=DEV)
            vf = torch.randn(B, Hkv, max(n, 1), D, generator=g, device=DEV)
            if kv == "int8":
                ki, ks = syn.quantize_per_vector(kf, torch.float32)
                vi, vs = syn.quantize_per_vector(vf, torch.float32)
                tensors = [q, ki, vi, ks, vs]
            else:
                tensors = [q, kf.to(torch.bfloat16), vf.to(torch.bfloat16)]
        kl = torch.full((1,), n, dtype=torch.int32, device=DEV)
        out = torch.full((B, 1, Hq, D), float("nan"), dtype=torch.bfloat16, device=DEV)
        ws = torch.empty(gpu_pkg.decode_workspace_size(B, Hq, Hkv, D), dtype=torch.uint8, device=DEV)
        ds = [L.desc(t) for t in tensors] + [L.desc(kl)]
        tail = [ctypes.c_float(D ** -0.5), ctypes.byref(L.desc(out)), ctypes.c_void_p(ws.data_ptr()),
                ctypes.c_size_t(ws.numel()), None, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)]
        if paged:
            fn = h.sia_paged_gqa_int8_flash_decode if kv == "int8" else h.sia_paged_attention_flash_decode
            rc = fn(*[ctypes.byref(d) for d in ds], ctypes.c_int32(16), *tail)
        else:
            fn = h.sia_attention_flash_decode_int8 if kv == "int8" else h.sia_attention_flash_decode
            rc = fn(*[ctypes.byref(d) for d in ds], *tail)
        assert rc == 0, h.sia_last_error_message()
        torch.cuda.synchronize()
        if n == 0:
            assert bool((out == 0).all()), "a zero length must give zero rows"
            continue
        if paged:
            if kv == "int8":
                ref = O.paged_int8_decode(f64(q), case.k_pool.cpu().numpy(), case.v_pool.cpu().numpy(),
                                          f64(case.k_scale), f64(case.v_scale), case.block_table.cpu().numpy(),
                                          [n] * B, 16)
            else:
                ref = O.paged_decode(f64(q), f64(case.k_pool), f64(case.v_pool), case.block_table.cpu().numpy(),
                                     [n] * B, 16)
        elif kv == "int8":
            ref = O.int8_decode(f64(q), ki.cpu().numpy(), vi.cpu().numpy(), f64(ks), f64(vs), [n] * B)
        else:
            ref = O.gqa_decode(f64(q), f64(tensors[1]), f64(tensors[2]), [n] * B)
        assert_close(out, ref, 1e-2 if kv == "int8" else 2e-3, f"shared length {n}")
