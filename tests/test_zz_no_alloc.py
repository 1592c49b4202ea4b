"""The no-allocation decode entry point against the workspace one, through the C ABI.

``sia_paged_gqa_int8_flash_decode_noalloc`` runs the kernels of
``sia_paged_gqa_int8_flash_decode`` with the library's static split-K scratch
in place of a caller workspace; both are called here through ctypes on the
same inputs and must agree bit for bit (the integer/byte bar: the same
kernels, the same split), on two calls in a row, the second with a smaller
batch and shorter contexts (the scratch keeps the first call's contents).
Both calls are also checked against the float64 oracle at the int8 bar.
"""

from __future__ import annotations

import ctypes
import importlib

import numpy as np
import pytest
import torch

from oracle import attention as O
from helpers import announce, assert_close, f64

pytestmark = pytest.mark.gpu

DEV = "cuda"
syn = importlib.import_module("simple-inference-autoresearch_amd.synthetic")
L = importlib.import_module("simple-inference-autoresearch_amd._lib")


def _call(h, name, case, out, ws=None):
    ds = [L.desc(t) for t in (case.q, case.k_pool, case.v_pool, case.k_scale, case.v_scale, case.block_table,
                              case.kv_len)]
    do = L.desc(out)
    scale = ctypes.c_float(1.0 / case.q.shape[-1] ** 0.5)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [ctypes.byref(d) for d in ds] + [ctypes.c_int32(case.page_size), scale, ctypes.byref(do)]
    if ws is not None:
        args += [ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(ws.numel())]
    rc = getattr(h, name)(*args, None, stream)
    assert rc == 0, (name, rc, h.sia_last_error_message())


def test_noalloc_matches_workspace_entry_point(gpu_pkg):
    h = L.require_library()
    cases = [
        ("B48 ragged 32/8 D128", [3000, 1, 8192, 517] * 12, 32, 8, 128, 21),
        ("B5 short 64/8 D128 (smaller second call)", [100, 33, 1, 700, 16], 64, 8, 128, 22),
    ]
    for label, ctx, Hq, Hkv, D, seed in cases:
        announce(f"no-alloc decode vs workspace decode: {label}")
        case = syn.paged_case(ctx, Hq=Hq, Hkv=Hkv, D=D, page=16, seed=seed, device=DEV, kv="int8")
        B = len(ctx)
        ws = torch.empty(gpu_pkg.decode_workspace_size(B, Hq, Hkv, D), dtype=torch.uint8, device=DEV)
        ref_out = torch.empty(B, 1, Hq, D, dtype=case.q.dtype, device=DEV)
        got = torch.full((B, 1, Hq, D), float("nan"), dtype=case.q.dtype, device=DEV)
        _call(h, "sia_paged_gqa_int8_flash_decode", case, ref_out, ws)
        _call(h, "sia_paged_gqa_int8_flash_decode_noalloc", case, got)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref_out.view(torch.int16)), f"{label}: outputs differ"
        ref = O.paged_int8_decode(f64(case.q), case.k_pool.cpu().numpy(), case.v_pool.cpu().numpy(),
                                  f64(case.k_scale), f64(case.v_scale), case.block_table.cpu().numpy(), ctx, 16)
        assert_close(got, ref, 1e-2, f"{label} vs oracle")


def test_noalloc_rejects_bad_arguments(gpu_pkg):
    """Validation errors of the workspace entry point carry over (no launch)."""
    h = L.require_library()
    case = syn.paged_case([64, 64], Hq=8, Hkv=2, D=128, page=16, seed=3, device=DEV, kv="int8")
    out = torch.empty(2, 1, 8, 128, dtype=case.q.dtype, device=DEV)
    ds = [L.desc(t) for t in (case.q, case.k_pool, case.v_pool, case.k_scale, case.v_scale)]
    dout = L.desc(out)
    rc = h.sia_paged_gqa_int8_flash_decode_noalloc(*[ctypes.byref(d) for d in ds], None,
                                                    ctypes.byref(L.desc(case.kv_len)), ctypes.c_int32(16),
                                                    ctypes.c_float(0.1), ctypes.byref(dout), None, None)
    assert rc == -1 and b"block_table" in h.sia_last_error_message()
