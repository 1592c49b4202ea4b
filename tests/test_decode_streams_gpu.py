"""Decode calls in sequence, in graphs and on several streams.

The split-K pieces of a call live in its workspace (taken per call from
torch's caching allocator, stream-ordered) and are merged by the merge kernel
on the same stream.  Checked against the float64 oracle (16-bit: 2e-3 before
one output rounding; int8: 1e-2, and 2e-3) and for bit-equality between runs:

* one long sequence (each KV head's work split over tens of work-groups);
* empty sequences between split ones, whose rows are written as zeros, into a
  NaN-filled output through the C ABI;
* the same call repeated on one stream, with calls of another geometry
  between: bit-equal outputs;
* one HIP graph holding three decode calls on one stream, replayed with eager
  calls between the replays: every replay bit-equal to the eager result;
* calls issued on two streams at once.
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


def oracle(case):
    if case.is_int8:
        return O.paged_int8_decode(f64(case.q), case.k_pool.cpu().numpy(), case.v_pool.cpu().numpy(),
                                   f64(case.k_scale), f64(case.v_scale), case.block_table.cpu().numpy(),
                                   case.ctx, case.page_size)
    return O.paged_decode(f64(case.q), f64(case.k_pool), f64(case.v_pool), case.block_table.cpu().numpy(),
                          case.ctx, case.page_size)


def run(pkg, case):
    if case.is_int8:
        return pkg.paged_gqa_int8_flash_decode(case.q, case.k_pool, case.v_pool, case.k_scale, case.v_scale,
                                               case.block_table, case.kv_len, case.page_size)
    return pkg.paged_attention_flash_decode(case.q, case.k_pool, case.v_pool, case.block_table, case.kv_len,
                                            case.page_size)


def check(out, case, what):
    ref = oracle(case)
    if case.is_int8:
        assert_close(out, ref, 1e-2, what)
    assert_close(out, ref, 2e-3, what)


@pytest.mark.parametrize("kv", ["bf16", "int8"])
def test_one_long_sequence(gpu_pkg, kv):
    """B1 x 32768 tokens, 32/8 heads: every KV head's work is split over tens of
    work-groups, and the merge kernel splits a row's pieces over its waves."""
    announce(f"decode one long sequence {kv}")
    case = syn.paged_case([32768], Hq=32, Hkv=8, D=128, page=16, seed=3, device=DEV, kv=kv)
    out = run(gpu_pkg, case)
    torch.cuda.synchronize()
    check(out, case, "one sequence")


def test_empty_sequences_into_nan_output(gpu_pkg):
    """Per-sequence lengths with empty sequences between split ones, through the C
    ABI into a NaN-filled output: every row is written, the empty ones as zeros."""
    h = L.require_library()
    announce("decode: empty sequences, NaN-filled output")
    ctx = [0, 2500, 0, 0, 900, 0]
    case = syn.paged_case(ctx, Hq=32, Hkv=8, D=128, page=16, seed=5, device=DEV, kv="bf16")
    B, Hq, D = len(ctx), 32, 128
    out = torch.full((B, 1, Hq, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(gpu_pkg.decode_workspace_size(B, Hq, 8, D), dtype=torch.uint8, device=DEV)
    ds = [L.desc(t) for t in (case.q, case.k_pool, case.v_pool, case.block_table, case.kv_len)]
    rc = h.sia_paged_attention_flash_decode(*[ctypes.byref(d) for d in ds], ctypes.c_int32(16),
                                            ctypes.c_float(D ** -0.5), ctypes.byref(L.desc(out)),
                                            ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(ws.numel()), None,
                                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, h.sia_last_error_message()
    torch.cuda.synchronize()
    for b in (0, 2, 3, 5):
        assert bool((out[b] == 0).all()), f"sequence {b} is empty: its rows must be zero"
    check(out, case, "C ABI, empty sequences")


def test_calls_in_a_row(gpu_pkg):
    """The same call gives bit-equal outputs each time, also after calls of another
    geometry on the same stream (nothing of one call leaks into the next)."""
    announce("decode: calls in a row")
    a = syn.paged_case([5000, 300, 2222], Hq=32, Hkv=8, D=128, page=16, seed=8, device=DEV, kv="int8")
    b = syn.paged_case([40, 9000, 1, 77, 4000], Hq=64, Hkv=8, D=128, page=16, seed=9, device=DEV, kv="bf16")
    first = run(gpu_pkg, a)
    torch.cuda.synchronize()
    check(first, a, "first call")
    for i in range(4):
        again = run(gpu_pkg, a)
        other = run(gpu_pkg, b)
        torch.cuda.synchronize()
        assert torch.equal(again, first), f"call {i + 2} differs from the first"
        check(other, b, f"other geometry, round {i}")


def test_graph_with_several_decode_calls(gpu_pkg):
    """Three decode calls captured on one stream, replayed five times with eager
    calls of the same shapes between the replays: every replay equals the eager
    outputs bit for bit."""
    announce("decode: graph of three decode calls")
    cases = [syn.paged_case(ctx, Hq=32, Hkv=8, D=128, page=16, seed=20 + i, device=DEV, kv=kv)
             for i, (ctx, kv) in enumerate((([3000, 100, 7000], "int8"), ([64, 4096], "bf16"),
                                            ([1, 2, 12000, 5], "int8")))]
    eager = [run(gpu_pkg, c) for c in cases]
    torch.cuda.synchronize()
    for c, o in zip(cases, eager):
        check(o, c, "eager")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):           # warm the allocator on the capture stream
        [run(gpu_pkg, c) for c in cases]
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [run(gpu_pkg, c) for c in cases]
    for r in range(5):
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), f"replay {r}, call {i}"
        between = [run(gpu_pkg, c) for c in cases]     # eager calls on the default stream in between
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(between, eager)):
            assert torch.equal(o, e), f"eager call {i} after replay {r}"


def test_two_streams_at_once(gpu_pkg):
    """Calls issued on two streams without synchronisation between them both
    match their single-stream results bit for bit."""
    announce("decode: two streams")
    a = syn.paged_case([9000, 3000, 500] * 4, Hq=32, Hkv=8, D=128, page=16, seed=30, device=DEV, kv="int8")
    b = syn.paged_case([12000, 40, 8000] * 3, Hq=32, Hkv=8, D=128, page=16, seed=31, device=DEV, kv="bf16")
    ref_a, ref_b = run(gpu_pkg, a), run(gpu_pkg, b)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs_a, outs_b = [], []
    for _ in range(6):
        with torch.cuda.stream(s1):
            outs_a.append(run(gpu_pkg, a))
        with torch.cuda.stream(s2):
            outs_b.append(run(gpu_pkg, b))
    torch.cuda.synchronize()
    for i in range(6):
        assert torch.equal(outs_a[i], ref_a), f"stream 1 call {i}"
        assert torch.equal(outs_b[i], ref_b), f"stream 2 call {i}"
    check(ref_a, a, "stream reference a")
    check(ref_b, b, "stream reference b")
