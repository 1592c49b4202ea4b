"""GPU parity of the fused RoPE kernel (``sia_rope_qk``) against the CPU oracle.

Bar: bit-exact against ``oracle.rope.rope_qk`` (fp32 math, every product and
sum rounded, output rounded to nearest even), the restatement of
``kernels/rope_kernel.py:86-165`` pinned by ``tests/test_oracle_rope.py``.
Cases follow the reference's own RoPE checks
(``workspace/scripts/parity_rope_strided_jun27.py``: strided qkv slices at
T = 1, 7, 29 equal to the contiguous path; ``benchmarks/bench_rope.py``:
Llama 3 tables) plus both pair layouts, both table widths, every float
dtype, head dims on the 16-byte path and the one-pair path, misaligned
inputs, decode tables of one row and empty inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import announce
from oracle import rope as OR

pytestmark = pytest.mark.gpu
DEV = "cuda"
_NP_DT = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}


def host(t):
    return t.detach().float().cpu().numpy()


def make_tables(Tc, D, dtype, width, start=0, theta=10000.0):
    inv = 1.0 / theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = torch.outer(torch.arange(start, start + Tc, dtype=torch.float64), inv)
    c, s = ang.cos(), ang.sin()
    if width == D:
        c, s = torch.cat([c, c], -1), torch.cat([s, s], -1)
    return c.to(dtype).to(DEV), s.to(dtype).to(DEV)


def check(pkg, q, k, cos, sin, interleaved, what):
    announce(f"rope {what}")
    gq, gk = pkg.rope_triton(q, k, cos, sin, interleaved=interleaved)
    torch.cuda.synchronize()
    assert gq.shape == q.shape and gk.shape == k.shape and gq.is_contiguous() and gk.is_contiguous()
    assert gq.dtype == q.dtype and gk.dtype == k.dtype
    rq, rk = OR.rope_qk(host(q), host(k), host(cos), host(sin), interleaved=interleaved, dtype=_NP_DT[q.dtype])
    hq, hk = host(gq), host(gk)
    assert np.array_equal(hq, rq), f"{what}: q differs at {np.argwhere(hq != rq)[:4].tolist()}"
    assert np.array_equal(hk, rk), f"{what}: k differs at {np.argwhere(hk != rk)[:4].tolist()}"
    return gq, gk


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [16, 64, 96, 128, 256, 10, 72])
@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_dtypes_dims_layouts(gpu_pkg, dtype, D, interleaved):
    torch.manual_seed(D)
    B, T, Hq, Hkv = 2, 9, 4, 2
    q = torch.randn(B, T, Hq, D, device=DEV).to(dtype)
    k = torch.randn(B, T, Hkv, D, device=DEV).to(dtype)
    for width in (D, D // 2):
        cos, sin = make_tables(T, D, dtype, width, start=3)
        check(gpu_pkg, q, k, cos, sin, interleaved, f"{dtype} D={D} il={interleaved} width={width}")


@pytest.mark.parametrize("qdt,cdt", [(torch.bfloat16, torch.float32), (torch.float16, torch.bfloat16),
                                     (torch.float32, torch.float16)])
def test_rope_table_dtype_differs(gpu_pkg, qdt, cdt):
    torch.manual_seed(5)
    q = torch.randn(3, 5, 8, 128, device=DEV).to(qdt)
    k = torch.randn(3, 5, 2, 128, device=DEV).to(qdt)
    cos, sin = make_tables(5, 128, cdt, 128)
    check(gpu_pkg, q, k, cos, sin, False, f"q {qdt} cos {cdt}")


@pytest.mark.parametrize("T", [1, 7, 29])
def test_rope_strided_qkv_slices(gpu_pkg, T):
    """Q/K slices of a fused qkv buffer: rotated in place of a copy, equal to the contiguous path."""
    torch.manual_seed(T)
    B, Hq, Hkv, D = 16, 32, 8, 128
    qs, ks = Hq * D, Hkv * D
    qkv = torch.randn(B, T, qs + 2 * ks, device=DEV, dtype=torch.bfloat16)
    q = qkv[..., :qs].reshape(B, T, Hq, D)
    k = qkv[..., qs:qs + ks].reshape(B, T, Hkv, D)
    assert not q.is_contiguous()
    cos = torch.randn(T, D, device=DEV, dtype=torch.bfloat16)
    sin = torch.randn(T, D, device=DEV, dtype=torch.bfloat16)
    gq, gk = check(gpu_pkg, q, k, cos, sin, False, f"qkv slices T={T}")
    cq, ck = gpu_pkg.rope_triton(q.contiguous(), k.contiguous(), cos, sin)
    assert torch.equal(gq, cq) and torch.equal(gk, ck)


def test_rope_non_flattenable_view_is_copied(gpu_pkg):
    # (B, H, T, D) transposed to (B, T, H, D): heads are not head_dim apart -> the wrapper copies
    q = torch.randn(2, 4, 6, 64, device=DEV, dtype=torch.bfloat16).transpose(1, 2)
    k = torch.randn(2, 1, 6, 64, device=DEV, dtype=torch.bfloat16).transpose(1, 2)
    cos, sin = make_tables(6, 64, torch.bfloat16, 64)
    check(gpu_pkg, q, k, cos, sin, False, "transposed view")
    # a single sequence whose batch stride is arbitrary (size-1 dims' strides are never used)
    base = torch.randn(6 * 8 * 64 + 64, device=DEV, dtype=torch.bfloat16)
    q1 = base.as_strided((1, 6, 4, 64), (7, 8 * 64, 64, 1))
    k1 = base.as_strided((1, 6, 1, 64), (3, 8 * 64, 5, 1), 4 * 64)
    check(gpu_pkg, q1, k1, cos, sin, False, "B=1 odd batch stride, H=1 odd head stride")


def test_rope_misaligned_inputs_take_scalar_path(gpu_pkg):
    torch.manual_seed(3)
    buf = torch.randn(2 * 3 * 4 * 64 + 1, device=DEV, dtype=torch.bfloat16)
    q = buf[1:].view(2, 3, 4, 64)                      # 2-byte offset: not 16-byte aligned
    k = torch.randn(2, 3, 2, 64, device=DEV, dtype=torch.bfloat16)
    cos, sin = make_tables(3, 64, torch.bfloat16, 64)
    check(gpu_pkg, q, k, cos, sin, False, "misaligned q")
    check(gpu_pkg, q, k, cos, sin, True, "misaligned q interleaved")


def test_rope_decode_one_row_table(gpu_pkg):
    """Decode: T == 1 with a one-row table at the current position serves every sequence."""
    torch.manual_seed(11)
    rf = gpu_pkg.RopeFrequencies(128, 4096, device=torch.device(DEV))
    cos, sin = rf.get(1, start_pos=4000, dtype=torch.bfloat16)
    q = torch.randn(64, 1, 32, 128, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(64, 1, 8, 128, device=DEV, dtype=torch.bfloat16)
    check(gpu_pkg, q, k, cos, sin, False, "decode B=64 pos=4000")


def test_rope_table_longer_than_rows(gpu_pkg):
    """Row r reads table row r % Tc also when the table has more rows than q has tokens."""
    torch.manual_seed(12)
    q = torch.randn(2, 3, 2, 64, device=DEV, dtype=torch.float16)
    k = torch.randn(2, 3, 1, 64, device=DEV, dtype=torch.float16)
    cos, sin = make_tables(5, 64, torch.float16, 32)
    check(gpu_pkg, q, k, cos, sin, False, "Tc=5 rows=6")


def test_rope_llama3_prefill_full_size(gpu_pkg):
    """The bench workload: Llama-3-8B heads, T = 8192, Llama 3 tables."""
    torch.manual_seed(13)
    rf = gpu_pkg.RopeFrequencies(128, 8192, device=torch.device(DEV))
    cos, sin = rf.get(8192, dtype=torch.bfloat16)
    q = torch.randn(1, 8192, 32, 128, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(1, 8192, 8, 128, device=DEV, dtype=torch.bfloat16)
    check(gpu_pkg, q, k, cos, sin, False, "llama3 T=8192")


def test_rope_empty_and_kv_only(gpu_pkg):
    cos, sin = make_tables(4, 64, torch.bfloat16, 64)
    q = torch.empty(0, 4, 2, 64, device=DEV, dtype=torch.bfloat16)
    k = torch.empty(0, 4, 1, 64, device=DEV, dtype=torch.bfloat16)
    gq, gk = gpu_pkg.rope_triton(q, k, cos, sin)
    assert gq.shape == q.shape and gk.shape == k.shape
    q = torch.randn(1, 4, 2, 64, device=DEV, dtype=torch.bfloat16)
    k = torch.empty(1, 4, 0, 64, device=DEV, dtype=torch.bfloat16)
    check(gpu_pkg, q, k, cos, sin, False, "no kv heads")


def test_rope_invalid_arguments(gpu_pkg):
    q = torch.randn(1, 2, 2, 63, device=DEV, dtype=torch.bfloat16)
    with pytest.raises((AssertionError, ValueError)):
        gpu_pkg.rope_triton(q, q[:, :, :1], torch.zeros(2, 63, device=DEV), torch.zeros(2, 63, device=DEV))
    q = torch.randn(1, 2, 2, 64, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(1, 3, 1, 64, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        gpu_pkg.rope_triton(q, k, torch.zeros(2, 64, device=DEV), torch.zeros(2, 64, device=DEV))
    with pytest.raises(ValueError, match="dtypes differ"):
        gpu_pkg.rope_triton(q, q.float(), torch.zeros(2, 64, device=DEV), torch.zeros(2, 64, device=DEV))
    with pytest.raises(NotImplementedError, match="not supported"):
        qi = torch.zeros(1, 2, 2, 64, device=DEV, dtype=torch.int32)
        gpu_pkg.rope_triton(qi, qi, torch.zeros(2, 64, device=DEV), torch.zeros(2, 64, device=DEV))
