#!/usr/bin/env python
"""Benchmark of the MI355X attention hot path (one GPU).

Headline (BASELINE.json ``metric``): paged INT8-KV GQA decode, config 3 --
batch 64, 32 Q / 8 KV heads, head_dim 128, page 16, every context 8192,
int8 K/V with per-token-per-head fp32 scales, bf16 queries.  One step is one
decode call over the whole batch with every input already resident in HBM.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-others]

Prints ONE JSON line.  ``value`` is the achieved algorithmic HBM throughput of
the whole call (GB/s); ``roofline`` refers to the dominant kernel
(``decode_main``), timed with HIP events recorded by the library on the launch
stream around that kernel alone; ``cpu_baseline`` times the reference's CPU
torch path (restated in ``oracle/eager_path.py``) on a bounded sample of the
same workload.  ``other_configs`` carries configs 1, 2 and 5 (decode), 4
(prefill), the fused RoPE, the Qwen3.5 shapes and one-sequence shapes
(``small``: prefill at the reference benchmark's lengths, single-sequence
decode) measured the same way when available.
"""

from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
PKG_NAME = "simple-inference-autoresearch_amd"

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
METRIC = "paged INT8-KV GQA decode: µs/call + achieved HBM GB/s (% of peak), 1 GPU"


def _pkg():
    return importlib.import_module(PKG_NAME)


def _syn():
    return importlib.import_module(PKG_NAME + ".synthetic")


def run_decode(pkg, case):
    if case.is_int8:
        return pkg.paged_gqa_int8_flash_decode(case.q, case.k_pool, case.v_pool, case.k_scale, case.v_scale,
                                               case.block_table, case.kv_len, case.page_size)
    return pkg.paged_attention_flash_decode(case.q, case.k_pool, case.v_pool, case.block_table, case.kv_len,
                                            case.page_size)


SETTLE_MS = 300.0   # set from --settle-ms


def settle(fn, ms: float | None = None) -> None:
    """Run `fn` back to back for about `ms` of wall time before any warm-up.

    An idle MI355X takes tens of milliseconds of sustained load to reach its
    steady clocks (a prefill kernel measured 193 us over its first launches
    and 153 us once settled), so short runs would time the ramp rather than
    the kernel.  This is untimed and separate from the W warm-up steps.
    """
    import torch

    budget = (SETTLE_MS if ms is None else ms) / 1e3
    if budget <= 0:
        return
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def time_decode(pkg, cases, steps: int, warmup: int):
    """Clock settle, W untimed calls, then two timed passes of exactly `steps` calls.

    Call i reads input set i % len(cases) (several sets rotate when one set
    would fit in the 256 MB MALL).  Pass 1: the library stamps a pair of HIP
    events with the start and end of `decode_main` of every call (launched
    through hipExtLaunchKernel, so the events are the dispatch's own
    timestamps, with no marker packets); main-kernel time = end_i - begin_i,
    whole-call time = begin_{i+1} - begin_i (main kernel, split-K merge and
    launch gaps; the last call is closed by one more call's begin).  Pass 2: no events between calls,
    only around the loop: the back-to-back mean per call and the host
    microseconds to issue one call.
    Returns (per-call whole-call ms, per-call main-kernel ms, back-to-back ms, host us).
    """
    import torch

    n = len(cases)
    settle(lambda: [run_decode(pkg, c) for c in cases])
    for i in range(warmup):
        run_decode(pkg, cases[i % n])
    begins = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    for e in begins + ends:   # create the underlying hipEvents before handing them to the library
        e.record()
    torch.cuda.synchronize()
    for i in range(steps + 1):
        with pkg.decode_options(main_events=(begins[i], ends[i])):
            run_decode(pkg, cases[i % n])
    torch.cuda.synchronize()
    calls = [begins[i].elapsed_time(begins[i + 1]) for i in range(steps)]
    kern = [begins[i].elapsed_time(ends[i]) for i in range(steps)]
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    h0 = time.perf_counter()
    for i in range(steps):
        run_decode(pkg, cases[i % n])
    host_us = (time.perf_counter() - h0) / steps * 1e6
    e1.record()
    torch.cuda.synchronize()
    return calls, kern, e0.elapsed_time(e1) / steps, host_us


def cpu_baseline(case, target_s: float):
    """Time the reference's CPU path (gather pages, dequantise, repeat_interleave + SDPA).

    Bounded sample: a few whole sequences of the same batch are copied to the
    host and run repeatedly for about `target_s` seconds; the reported rate is
    the same algorithmic-bytes metric over the sequences processed.
    """
    import torch

    from oracle import eager_path as E

    rows = [0, 1, 2, 3]
    B, Hq, _, D = case.q.shape
    Hkv, page = case.k_pool.shape[1], case.page_size
    # pull just these sequences' pages to the host and renumber them
    pages, bts = [], []
    base = 0
    for r in rows:
        n = math.ceil(case.ctx[r] / page)
        pages.append(case.block_table[r, :n].long())
        bts.append(torch.arange(base, base + n, dtype=torch.int32))
        base += n
    idx = torch.cat(pages)
    kp, vp = case.k_pool[idx].cpu(), case.v_pool[idx].cpu()
    ksp, vsp = case.k_scale[idx].cpu(), case.v_scale[idx].cpu()
    maxn = max(len(b) for b in bts)
    bt = torch.zeros(len(rows), maxn, dtype=torch.int32)
    for i, b in enumerate(bts):
        bt[i, :len(b)] = b
    q = case.q[rows].float().cpu()
    lens = [case.ctx[r] for r in rows]
    sub_rows = list(range(len(rows)))
    for _ in range(2):  # warm-up
        E.eager_paged_int8_decode(q, kp, vp, ksp, vsp, bt, lens, page, batch_rows=sub_rows)
    reps, t_start = 0, time.perf_counter()
    times = []
    while True:
        t = time.perf_counter()
        E.eager_paged_int8_decode(q, kp, vp, ksp, vsp, bt, lens, page, batch_rows=sub_rows)
        times.append(time.perf_counter() - t)
        reps += 1
        if time.perf_counter() - t_start >= target_s and reps >= 5:
            break
    tokens = sum(lens)
    sample_bytes = (tokens * Hkv * D * 2 + tokens * Hkv * 4 * 2 + 2 * len(rows) * Hq * D * 2
                    + 4 * sum(len(b) for b in bts))
    med = statistics.median(times)
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except (OSError, StopIteration):
        model = platform.processor()
    return {
        "value": round(sample_bytes / med / 1e9, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"config-3 sequences {rows} ({tokens} tokens, {sample_bytes} algorithmic bytes) through "
                   f"oracle/eager_path.py (gather pages, dequantise, repeat_interleave + SDPA, fp32), "
                   f"median of {reps} reps over {time.perf_counter() - t_start:.1f}s"),
        "us_per_sample": round(med * 1e6, 1),
        "host_cpu": model,
        "os_cpu_count": os.cpu_count(),
    }


MALL_BYTES = 256 << 20   # MI355X Infinity Cache


def bench_decode_config(pkg, cases, steps, warmup):
    syn = _syn()
    calls, kern, ms, host_us = time_decode(pkg, cases, steps, warmup)
    nbytes = syn.decode_bytes(cases[0])
    k_med, c_med = statistics.median(kern), statistics.median(calls)
    gbs = lambda t_ms: round(nbytes / (t_ms * 1e-3) / 1e9, 1)
    return {
        "us_per_call": round(c_med * 1e3, 2),
        "us_per_call_min": round(min(calls) * 1e3, 2),
        "us_per_call_back_to_back": round(ms * 1e3, 2),
        "GBps": gbs(ms),
        "GBps_median_call": gbs(c_med),
        "main_kernel_us": round(k_med * 1e3, 2),
        "main_kernel_us_min": round(min(kern) * 1e3, 2),
        "main_kernel_us_mean": round(statistics.mean(kern) * 1e3, 2),
        "main_kernel_GBps": gbs(k_med),
        "frac_of_hbm_peak": round(nbytes / (k_med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "host_us_per_call": round(host_us, 2),
        "input_sets": len(cases),
        "input_bytes_total": sum(syn.decode_bytes(c) for c in cases),
        "algorithmic_bytes": nbytes,
        "statistic": (f"GBps and back_to_back: the {steps} timed calls issued back to back between two "
                      "synchronizes (no events between calls); us_per_call: median of a separate pass of "
                      f"{steps} calls, begin-to-begin of the events stamped with decode_main's start (min "
                      "alongside)"),
    }


def config_cases(syn, name, dev):
    """Input sets of a decode config: one when it exceeds the MALL twice over, else at
    least 4 (over 512 MB together) with the same lengths and shapes but other data and
    page maps, so that no call finds its K/V in the MALL."""
    first = getattr(syn, name)(dev)
    nbytes = syn.decode_bytes(first)
    if nbytes > 2 * MALL_BYTES:
        return [first]
    n = max(4, math.ceil(2 * MALL_BYTES / nbytes))
    return [first] + [syn.config_variant(name, dev, i) for i in range(1, n)]


def bench_prefill_config(pkg, steps: int, warmup: int):
    """Config 4: causal bf16 prefill B4 T2048 32/8 heads D128 -> MFMA TFLOP/s (T^2/2 FLOP convention)."""
    import torch

    syn = _syn()
    q, k, v = syn.cfg4(torch.device("cuda:0"))
    B, Hq, T, D = q.shape
    t = time_calls(lambda: pkg.attention_flash_triton(q, k, v, causal=True, out_token_major=True), steps, warmup)
    flops = syn.prefill_flops(B, Hq, T, D)
    tf = flops / (t["mean_ms"] * 1e-3) / 1e12
    tf_med = flops / (t["median_ms"] * 1e-3) / 1e12
    return {**_timing_fields(t), "TFLOPs": round(tf, 1), "frac_of_bf16_mfma_peak": round(tf / BF16_PEAK_TFLOPS, 4),
            "TFLOPs_median_call": round(tf_med, 1),
            "algorithmic_flops": flops, "workload": "config 4: causal prefill bf16 B4 T2048 32/8 heads D128",
            "statistic": (f"TFLOPs: the {steps} timed calls issued back to back between two synchronizes (as the "
                          f"headline's value); TFLOPs_median_call: median of a separate pass of {steps} calls "
                          "with an event between calls"),
            "rope_prologue": bench_rope_prologue(pkg, q, k, v, steps, warmup),
            "fp16_same_shape": bench_prefill_f16(pkg, q, k, v, steps, warmup)}


def bench_prefill_f16(pkg, q, k, v, steps: int, warmup: int):
    """The config-4 shape in float16, whose V the kernel reads in place (no V repack
    launch); same 2.5 PFLOP/s dense peak."""
    import torch

    qh, kh, vh = (t.to(torch.float16) for t in (q, k, v))
    B, Hq, T, D = q.shape
    t = time_calls(lambda: pkg.attention_flash_triton(qh, kh, vh, causal=True, out_token_major=True), steps, warmup)
    tf = _syn().prefill_flops(B, Hq, T, D) / (t["mean_ms"] * 1e-3) / 1e12
    return {"us_per_call": round(t["median_ms"] * 1e3, 2), "us_per_call_back_to_back": round(t["mean_ms"] * 1e3, 2),
            "TFLOPs": round(tf, 1), "frac_of_fp16_mfma_peak": round(tf / BF16_PEAK_TFLOPS, 4)}


def bench_rope_prologue(pkg, q, k, v, steps: int, warmup: int):
    """The same prefill with q rotated as it is loaded (rope_attention_flash_triton) against
    the reference's order for q: rope_triton, then attention on the rotated copy.  q is
    token-major (B, T, Hq, D), as the qkv projection leaves it, so both read it in place;
    K is taken as already rotated in both (the cache write rotates it)."""
    B, Hq, T, D = q.shape
    rf = pkg.RopeFrequencies(D, T, device=q.device)
    cos, sin = rf.get(T, start_pos=0, dtype=q.dtype)
    q_tm = q.transpose(1, 2).contiguous()
    k1 = q_tm[:, :, :1]        # rope_triton rotates a k as well: one head, negligible

    def unfused():
        qr, _ = pkg.rope_triton(q_tm, k1, cos, sin)
        return pkg.attention_flash_triton(qr.transpose(1, 2), k, v, causal=True, out_token_major=True)

    fused = time_calls(lambda: pkg.rope_attention_flash_triton(q_tm.transpose(1, 2), k, v, cos, sin, causal=True,
                                                                out_token_major=True), steps, warmup)
    sep = time_calls(unfused, steps, warmup)
    return {"fused_us_per_call": round(fused["median_ms"] * 1e3, 2),
            "rope_then_attention_us_per_call": round(sep["median_ms"] * 1e3, 2),
            "fused_us_per_call_back_to_back": round(fused["mean_ms"] * 1e3, 2),
            "rope_then_attention_us_per_call_back_to_back": round(sep["mean_ms"] * 1e3, 2),
            "statistic": f"us_per_call: median of {steps} calls each; back_to_back: mean of {steps} calls issued "
                         "back to back"}


def bench_config1(pkg, steps: int, warmup: int):
    """Config 1 on the GPU: contiguous fp32 decode B1, 32/8 heads, D64, ctx 512 (seed 0),
    scale 1/8, through attention_flash_decode (the fp32 vector-ALU path)."""
    import torch

    dev = torch.device("cuda:0")
    q, k, v = (t.to(dev) for t in _syn().cfg1())
    kv_len = torch.tensor([512], dtype=torch.int32, device=dev)
    t = time_calls(lambda: pkg.attention_flash_decode(q, k, v, kv_len, 0.125), steps, warmup)
    nbytes = 2 * 8 * 512 * 64 * 4 + 2 * 32 * 64 * 4
    gbs = nbytes / (t["median_ms"] * 1e-3) / 1e9
    return {**_timing_fields(t), "GBps": round(gbs, 1), "algorithmic_bytes": nbytes,
            "workload": "config 1: contiguous fp32 decode B1 32/8 heads D64 ctx 512 (2.1 MB: launch-bound)"}


def rope_bytes(B: int, T: int, Hq: int, Hkv: int, D: int, es: int = 2) -> int:
    """Algorithmic bytes of one fused RoPE call: read q, k and one cos and one sin row per
    token, write q_rot, k_rot (the reference's convention,
    benchmarks/benchmark_kernel/bench_rope_compare.py:28-34)."""
    return (2 * B * T * (Hq + Hkv) * D + 2 * T * D) * es


def bench_rope_config(pkg, steps: int, warmup: int):
    """Fused q/k RoPE (bf16, Llama-3-8B heads 32/8, D128, Llama 3 tables): a long prefill
    (B1 T8192, HBM-bound) and a decode step (B64 T1, one table row)."""
    import torch

    dev = torch.device("cuda:0")
    rf = pkg.RopeFrequencies(128, 8192, device=dev)
    out = {}
    for label, B, T in (("prefill_B1_T8192", 1, 8192), ("decode_B64_T1", 64, 1)):
        g = torch.Generator(device=dev).manual_seed(7)
        q = torch.randn(B, T, 32, 128, device=dev, dtype=torch.bfloat16, generator=g)
        k = torch.randn(B, T, 8, 128, device=dev, dtype=torch.bfloat16, generator=g)
        cos, sin = rf.get(T, start_pos=0 if T > 1 else 4000, dtype=torch.bfloat16)
        t = time_calls(lambda: pkg.rope_triton(q, k, cos, sin), steps, warmup)
        nbytes = rope_bytes(B, T, 32, 8, 128)
        gbs = nbytes / (t["mean_ms"] * 1e-3) / 1e9
        out[label] = {**_timing_fields(t), "GBps": round(gbs, 1),
                      "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                      "GBps_median_call": round(nbytes / (t["median_ms"] * 1e-3) / 1e9, 1),
                      "algorithmic_bytes": nbytes}
    out["workload"] = "fused q/k RoPE bf16, 32/8 heads D128, split-half, Llama 3 tables"
    out["statistic"] = ("GBps: calls issued back to back between two synchronizes; GBps_median_call and the "
                        "*_us_per_call of rope_kv_write: median of a pass with an event between calls")
    out["rope_kv_write"] = bench_rope_kv_write(pkg, rf, steps, warmup)
    return out


def rope_kv_write_bytes(B: int, T: int, Hq: int, Hkv: int, D: int) -> int:
    """Algorithmic bytes of one fused RoPE + int8 KV write (bf16 q/k/v, bf16 tables, int8 K/V with
    fp32 scales): read q, k, v and half a cos and a sin row per token; write q_rot, the int8 K/V
    rows and their scales."""
    per_token = (Hq + 2 * Hkv) * D * 2 + 2 * (D // 2) * 2 + Hq * D * 2 + 2 * Hkv * D + 2 * Hkv * 4
    return B * T * per_token


def bench_rope_kv_write(pkg, rf, steps: int, warmup: int):
    """RoPE of q and k fused into the int8 cache write (one launch), against the reference's order
    (RoPE launch, then the write) on the same inputs: prefill B1 T8192 into a contiguous int8 cache,
    and a B64 decode step into paged int8 pools at per-sequence positions."""
    import torch

    dev = torch.device("cuda:0")
    Hq, Hkv, D = 32, 8, 128
    cos, sin = rf.get(8192, dtype=torch.bfloat16)
    out = {}
    for label, B, T in (("prefill_B1_T8192", 1, 8192), ("decode_B64_T1", 64, 1)):
        g = torch.Generator(device=dev).manual_seed(9)
        qkv = torch.randn(B, T, (Hq + 2 * Hkv) * D, device=dev, dtype=torch.bfloat16, generator=g)
        q = qkv[..., :Hq * D].view(B, T, Hq, D)
        k = qkv[..., Hq * D:(Hq + Hkv) * D].view(B, T, Hkv, D)
        v = qkv[..., (Hq + Hkv) * D:].view(B, T, Hkv, D)
        if T > 1:
            kc = torch.zeros(B, Hkv, 8192, D, dtype=torch.int8, device=dev)
            vc = torch.zeros_like(kc)
            ks = torch.zeros(B, Hkv, 8192, dtype=torch.float32, device=dev)
            vs = torch.zeros_like(ks)
            kw = dict(start_offset=0)
            cs, sn = cos, sin
        else:
            pages = B * 512
            kc = torch.zeros(pages, Hkv, 16, D, dtype=torch.int8, device=dev)
            vc = torch.zeros_like(kc)
            ks = torch.zeros(pages, Hkv, 16, dtype=torch.float32, device=dev)
            vs = torch.zeros_like(ks)
            bt = torch.randperm(pages, device=dev, generator=g).int().view(B, 512)
            pos = torch.randint(1, 8192, (B,), device=dev, generator=g).int()
            kw = dict(block_table=bt, start_pos=pos, start_offset=-1, page_size=16)
            cs, sn = cos, sin
        q_out = torch.empty(B, T, Hq, D, dtype=torch.bfloat16, device=dev)

        def fused():
            pkg.rope_kv_write(q, k, v, cs, sn, kc, vc, ks, vs, q_out=q_out, **kw)

        def unfused():   # the reference's order; shared position 0.. for prefill, row 4000 for decode
            if T > 1:
                qr, kr = pkg.rope_triton(q, k, cos, sin)
            else:
                qr, kr = pkg.rope_triton(q, k, cos[4000:4001], sin[4000:4001])
            pkg.kv_write(kr.transpose(1, 2), v.contiguous().transpose(1, 2), kc, vc, ks, vs, **kw)

        res = {}
        b2b = {}
        host = {}
        for name, fn in (("fused", fused), ("rope_then_write", unfused)):
            t = time_calls(fn, steps, warmup)
            res[name] = round(t["median_ms"] * 1e3, 2)
            b2b[name] = round(t["mean_ms"] * 1e3, 2)
            host[name] = round(t["host_us"], 2)
        nbytes = rope_kv_write_bytes(B, T, Hq, Hkv, D)
        gbs = nbytes / (b2b["fused"] * 1e-6) / 1e9
        out[label] = {"fused_us_per_call": res["fused"], "rope_then_write_us_per_call": res["rope_then_write"],
                      "fused_us_per_call_back_to_back": b2b["fused"],
                      "rope_then_write_us_per_call_back_to_back": b2b["rope_then_write"],
                      "fused_host_us_per_call": host["fused"],
                      "fused_GBps": round(gbs, 1), "fused_frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                      "algorithmic_bytes": nbytes}
    out["workload"] = ("RoPE of q, k fused into the int8 KV write (bf16 q/k/v slices of one qkv buffer, "
                       "32/8 heads D128, fp32 scales)")
    return out


def time_calls(fn, steps: int, warmup: int) -> dict:
    """Clock settle, W untimed calls, then two timed passes of `steps` back-to-back calls.

    Pass 1 records a HIP event on the current stream at every call boundary:
    the median and min milliseconds per call.  Pass 2 records events only
    around the whole loop: the mean milliseconds per call of an unbroken
    sequence of calls, and the host microseconds to issue one call (an event
    record itself costs the host about 4 us, so pass 1 overstates the wall
    time of calls whose kernels are shorter than their host cost)."""
    import torch

    settle(fn)
    for _ in range(warmup):
        fn()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    for i in range(steps):
        marks[i].record()
        fn()
    marks[steps].record()
    torch.cuda.synchronize()
    per = [marks[i].elapsed_time(marks[i + 1]) for i in range(steps)]
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    h0 = time.perf_counter()
    for _ in range(steps):
        fn()
    host_us = (time.perf_counter() - h0) / steps * 1e6
    e1.record()
    torch.cuda.synchronize()
    return {"median_ms": statistics.median(per), "min_ms": min(per),
            "mean_ms": e0.elapsed_time(e1) / steps, "host_us": host_us}


def _timing_fields(t: dict) -> dict:
    return {"us_per_call": round(t["median_ms"] * 1e3, 2), "us_per_call_min": round(t["min_ms"] * 1e3, 2),
            "us_per_call_back_to_back": round(t["mean_ms"] * 1e3, 2), "host_us_per_call": round(t["host_us"], 2)}


def bench_qwen35_config(pkg, steps: int, warmup: int):
    """Qwen3.5 full-attention shapes (head_dim 256, 16 query / 4 KV heads, bf16), the path the
    transformers attention hook takes: decode B32 over a contiguous 4096-token cache
    (attention_flash_decode) and a causal prefill of 4096 tokens (attention_flash_triton)."""
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(11)
    Hq, Hkv, D = 16, 4, 256
    out = {}
    B, S = 32, 4096
    q = torch.randn(B, Hq, 1, D, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, device=dev, generator=g).to(torch.bfloat16)
    kv_len = torch.tensor([S], dtype=torch.int32, device=dev)
    t = time_calls(lambda: pkg.attention_flash_decode(q, k, v, kv_len), steps, warmup)
    nbytes = 2 * B * Hkv * S * D * 2 + 2 * B * Hq * D * 2
    gbs = nbytes / (t["mean_ms"] * 1e-3) / 1e9
    out["decode_B32_ctx4096"] = {**_timing_fields(t), "GBps": round(gbs, 1),
                                 "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                                 "GBps_median_call": round(nbytes / (t["median_ms"] * 1e-3) / 1e9, 1),
                                 "algorithmic_bytes": nbytes}
    del q, k, v
    T = 4096
    q = (torch.randn(1, Hq, T, D, device=dev, generator=g) * 0.5).to(torch.bfloat16)
    k = (torch.randn(1, Hkv, T, D, device=dev, generator=g) * 0.5).to(torch.bfloat16)
    v = (torch.randn(1, Hkv, T, D, device=dev, generator=g) * 0.5).to(torch.bfloat16)
    t = time_calls(lambda: pkg.attention_flash_triton(q, k, v, causal=True, out_token_major=True), steps, warmup)
    flops = _syn().prefill_flops(1, Hq, T, D)
    tf = flops / (t["mean_ms"] * 1e-3) / 1e12
    out["prefill_B1_T4096"] = {**_timing_fields(t), "TFLOPs": round(tf, 1),
                               "frac_of_bf16_mfma_peak": round(tf / BF16_PEAK_TFLOPS, 4),
                               "TFLOPs_median_call": round(flops / (t["median_ms"] * 1e-3) / 1e12, 1),
                               "algorithmic_flops": flops}
    out["workload"] = "Qwen3.5 full attention: head_dim 256, 16/4 heads, bf16, contiguous cache"
    out["statistic"] = ("GBps / TFLOPs: calls issued back to back between two synchronizes; *_median_call: "
                        "median of a separate pass with an event between calls")
    return out


def bench_small_config(pkg, steps: int, warmup: int):
    """One sequence at a time (Llama-3.1-8B attention shapes: 32/8 heads, head_dim 128,
    bf16): causal prefill at the reference's own benchmark lengths
    (benchmarks/benchmark_kernel/bench_attention_compare.py:99-105, B1, T 128 .. 4096),
    the same prefill in fp16 at T 512 and 2048 (same 2.5 PFLOP/s dense peak), and
    decode over a contiguous cache of 8192 and 32768 tokens (bf16, and int8 with the
    fp16 scales of the reference's KVCache)."""
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(13)
    Hq, Hkv, D = 32, 8, 128
    out = {}
    for T in (128, 512, 1024, 2048, 4096):
        q = (torch.randn(1, Hq, T, D, device=dev, generator=g) * 0.5).to(torch.bfloat16)
        k = (torch.randn(1, Hkv, T, D, device=dev, generator=g) * 0.5).to(torch.bfloat16)
        v = (torch.randn(1, Hkv, T, D, device=dev, generator=g) * 0.5).to(torch.bfloat16)
        t = time_calls(lambda: pkg.attention_flash_triton(q, k, v, causal=True), steps, warmup)
        flops = _syn().prefill_flops(1, Hq, T, D)
        tf = flops / (t["mean_ms"] * 1e-3) / 1e12
        out[f"prefill_B1_T{T}"] = {**_timing_fields(t), "TFLOPs_back_to_back": round(tf, 1),
                                   "frac_of_bf16_mfma_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
    # float16 prefill (V read in place by transposed LDS reads, no V repack launch)
    for T in (512, 2048):
        q = (torch.randn(1, Hq, T, D, device=dev, generator=g) * 0.5).to(torch.float16)
        k = (torch.randn(1, Hkv, T, D, device=dev, generator=g) * 0.5).to(torch.float16)
        v = (torch.randn(1, Hkv, T, D, device=dev, generator=g) * 0.5).to(torch.float16)
        t = time_calls(lambda: pkg.attention_flash_triton(q, k, v, causal=True), steps, warmup)
        tf = _syn().prefill_flops(1, Hq, T, D) / (t["mean_ms"] * 1e-3) / 1e12
        out[f"prefill_f16_B1_T{T}"] = {**_timing_fields(t), "TFLOPs_back_to_back": round(tf, 1),
                                       "frac_of_fp16_mfma_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
    q = torch.randn(1, Hq, 1, D, device=dev, generator=g).to(torch.bfloat16)
    for S in (8192, 32768):
        kv_len = torch.tensor([S], dtype=torch.int32, device=dev)
        k = torch.randn(1, Hkv, S, D, device=dev, generator=g).to(torch.bfloat16)
        v = torch.randn(1, Hkv, S, D, device=dev, generator=g).to(torch.bfloat16)
        t = time_calls(lambda: pkg.attention_flash_decode(q, k, v, kv_len), steps, warmup)
        nbytes = 2 * Hkv * S * D * 2 + 2 * Hq * D * 2
        gbs = nbytes / (t["mean_ms"] * 1e-3) / 1e9
        out[f"decode_bf16_B1_ctx{S}"] = {**_timing_fields(t), "GBps_back_to_back": round(gbs, 1),
                                         "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        ki = torch.randint(-127, 128, (1, Hkv, S, D), device=dev, generator=g, dtype=torch.int8)
        vi = torch.randint(-127, 128, (1, Hkv, S, D), device=dev, generator=g, dtype=torch.int8)
        ks = (torch.rand(1, Hkv, S, device=dev, generator=g) * 0.02 + 1e-3).to(torch.float16)
        vs = (torch.rand(1, Hkv, S, device=dev, generator=g) * 0.02 + 1e-3).to(torch.float16)
        t = time_calls(lambda: pkg.attention_flash_decode_int8(q, ki, vi, ks, vs, kv_len), steps, warmup)
        nbytes = 2 * Hkv * S * (D + 2) + 2 * Hq * D * 2
        gbs = nbytes / (t["mean_ms"] * 1e-3) / 1e9
        out[f"decode_int8_B1_ctx{S}"] = {**_timing_fields(t), "GBps_back_to_back": round(gbs, 1),
                                         "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    out["workload"] = ("one sequence, 32/8 heads, head_dim 128, bf16: causal prefill at the reference "
                       "benchmark's lengths (and fp16 at two of them); decode over a contiguous cache "
                       "(rates from back-to-back calls)")
    return out


def bench_copy(steps: int, warmup: int, nbytes: int = 1 << 30):
    """A plain device-to-device copy of `nbytes` (torch's copy kernel).

    Reads and writes exactly `nbytes` per launch, so rocprofv3's FETCH_SIZE /
    WRITE_SIZE for it give the counters' scale against known HBM traffic; its
    rate is also the practically reachable streaming bandwidth.
    """
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(warmup):
        dst.copy_(src)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return {"bytes_read": nbytes, "bytes_written": nbytes, "us_per_call": round(ms * 1e3, 2),
            "GBps_read_plus_write": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}


def load_traffic(kernel: str):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE/WRITE_SIZE (profiles/), or None."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--settle-ms", type=float, default=300.0,
                   help="untimed back-to-back calls before each config's warm-up, so the GPU clocks settle")
    p.add_argument("--no-others", action="store_true", help="skip configs 2, 4, 5, the RoPE and the Qwen3.5 lines")
    p.add_argument("--config", default="cfg3", choices=["cfg2", "cfg3", "cfg4", "cfg5", "rope", "qwen35", "small", "copy"],
                   help="config to run alone (profiling runs); 'copy' is a plain 1 GiB device copy "
                        "that calibrates the HBM byte counters")
    args = p.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures the attention hot path on ONE GPU; multi-GPU runs are out of scope "
              "for this build (each GPU box has one MI355X). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    global SETTLE_MS
    SETTLE_MS = args.settle_ms
    pkg = _pkg()
    pkg.require_library()
    syn = _syn()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.config == "copy":   # counter calibration: 1 GiB read + 1 GiB written per launch
        r = bench_copy(args.steps, args.warmup)
        print(json.dumps({"config": "copy", **r}), flush=True)
        return 0
    if args.config == "small":   # one-sequence shapes only (profiling runs)
        r = bench_small_config(pkg, args.steps, args.warmup)
        print(json.dumps({"config": "small", **r}), flush=True)
        return 0
    if args.config == "qwen35":   # Qwen3.5 attention shapes only (profiling runs)
        r = bench_qwen35_config(pkg, args.steps, args.warmup)
        print(json.dumps({"config": "qwen35", **r}), flush=True)
        return 0
    if args.config == "rope":   # fused RoPE only (profiling runs)
        r = bench_rope_config(pkg, args.steps, args.warmup)
        print(json.dumps({"config": "rope", **r}), flush=True)
        return 0
    if args.config == "cfg4":   # prefill only (profiling runs)
        r = bench_prefill_config(pkg, args.steps, args.warmup)
        print(f"[bench] cfg4: {r}", file=sys.stderr, flush=True)
        print(json.dumps({"config": "cfg4", **r}), flush=True)
        return 0
    cases = config_cases(syn, args.config, dev)
    case = cases[0]
    torch.cuda.synchronize()
    print(f"[bench] {args.config}: inputs resident ({syn.decode_bytes(case)/1e9:.3f} GB algorithmic, "
          f"{len(cases)} rotating set(s))", file=sys.stderr, flush=True)
    head = bench_decode_config(pkg, cases, args.steps, args.warmup)
    print(f"[bench] {args.config}: {head}", file=sys.stderr, flush=True)

    result = {
        "metric": METRIC,
        "value": head["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_settle_ms": args.settle_ms,
        "ms_per_step": round(head["us_per_call_back_to_back"] / 1e3, 5),
        "us_per_call": head["us_per_call"],
        "us_per_call_min": head["us_per_call_min"],
        "us_per_call_back_to_back": head["us_per_call_back_to_back"],
        "host_us_per_call": head["host_us_per_call"],
        "statistic": head["statistic"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if case.is_int8 else "fp16",
        "dtype_detail": ("int8 K/V (QK on int8 MFMA, exact int32 dots), bf16 q/out, f16 PV MFMA, fp32 softmax/accumulate"
                         if case.is_int8 else "fp16 q/K/V/out, f16 MFMA, fp32 softmax/accumulate"),
        "data": ("synthetic (seeded N(0,1) K/V quantised per token per head; random page permutation)" if case.is_int8
                 else "synthetic (seeded N(0,1) q/K/V; random page permutation)"),
        "config": {
            "workload": {"cfg2": "config 2: paged fp16 decode B16 ctx U[256,4096]",
                         "cfg3": "config 3: paged INT8-KV GQA decode B64 ctx 8192",
                         "cfg5": "config 5: split-K paged INT8-KV decode B256 Hq64 lognormal ctx"}[args.config],
            "batch": int(case.q.shape[0]), "q_heads": int(case.q.shape[1]), "kv_heads": int(case.k_pool.shape[1]),
            "head_dim": int(case.q.shape[3]), "page_size": case.page_size, "contexts": f"sum {sum(case.ctx)}",
            "algorithmic_bytes": head["algorithmic_bytes"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": head["main_kernel_GBps"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": head["frac_of_hbm_peak"],
            "traffic": None,
            "kernel": "decode_main",
            "kernel_us": head["main_kernel_us"],
            "kernel_us_min": head["main_kernel_us_min"],
            "statistic": "median of the per-call HIP events stamped with decode_main's start and end",
        },
    }
    tr = load_traffic(f"decode_main_{args.config}")
    if tr is not None:
        result["roofline"]["traffic"] = tr.get("hbm_bytes_per_launch")
        result["roofline"]["traffic_source"] = tr.get("source")

    if not args.no_others and args.config == "cfg3":
        others = {}
        del case, cases
        torch.cuda.empty_cache()
        for name in ("cfg2", "cfg5"):
            cs = config_cases(syn, name, dev)
            torch.cuda.synchronize()
            others[name] = bench_decode_config(pkg, cs, max(50, args.steps // 2), args.warmup)
            print(f"[bench] {name}: {others[name]}", file=sys.stderr, flush=True)
            del cs
            torch.cuda.empty_cache()
        others["cfg1"] = bench_config1(pkg, max(50, args.steps // 2), args.warmup)
        print(f"[bench] cfg1: {others['cfg1']}", file=sys.stderr, flush=True)
        others["cfg4"] = bench_prefill_config(pkg, max(50, args.steps // 2), args.warmup)
        print(f"[bench] cfg4: {others['cfg4']}", file=sys.stderr, flush=True)
        others["rope"] = bench_rope_config(pkg, max(50, args.steps // 2), args.warmup)
        print(f"[bench] rope: {others['rope']}", file=sys.stderr, flush=True)
        others["qwen35"] = bench_qwen35_config(pkg, max(50, args.steps // 2), args.warmup)
        print(f"[bench] qwen35: {others['qwen35']}", file=sys.stderr, flush=True)
        others["small"] = bench_small_config(pkg, max(50, args.steps // 2), args.warmup)
        print(f"[bench] small: {others['small']}", file=sys.stderr, flush=True)
        result["other_configs"] = others
        case = None

    if not args.no_cpu_baseline:
        if case is None or not case.is_int8:   # the CPU baseline is the headline (config 3) path
            case = syn.cfg3(dev)
        print("[bench] timing the CPU baseline sample", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(case, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
