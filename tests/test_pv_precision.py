"""Why the prefill PV product takes P in f16 (CPU, float64 arithmetic model).

The causal prefill kernel rounds the softmax weights P to f16 and runs PV on
the f16 MFMA, with V converted to f16 once per call.  The reference rounds P
to V's dtype instead (``tl.dot(p.to(v.dtype), v)``,
``kernels/attention_kernel.py:221``), which for bf16 inputs is a bf16 P.  This
model of both roundings (fp32 weights, one rounding of P, the row sum over the
rounded weights as the kernel takes it, one bf16 output rounding) shows that a
bf16 P misses the 16-bit parity bar on ordinary N(0, 1) inputs, where the f16
P the kernel uses stays inside it.  That is the reason a transposed LDS read
of raw bf16 V rows (which would need a bf16 P) is not used for bf16 inputs.
"""

from __future__ import annotations

import numpy as np
import torch

from helpers import allowed_error


def _worst_ratio(p_dtype, T=256, D=128, heads=8, seed=1):
    g = torch.Generator().manual_seed(seed)
    worst = 0.0
    for _ in range(heads):
        q, k, v = (torch.randn(T, D, generator=g).to(torch.bfloat16).double().numpy() for _ in range(3))
        s = q @ k.T / np.sqrt(D)
        s[np.triu_indices(T, 1)] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        ref = (p @ v) / p.sum(1, keepdims=True)
        pr = torch.from_numpy(p.astype(np.float32)).to(p_dtype).double().numpy()
        o = torch.from_numpy((pr @ v) / pr.sum(1, keepdims=True)).to(torch.bfloat16).double().numpy()
        worst = max(worst, float((np.abs(o - ref) / allowed_error(ref, torch.bfloat16, 2e-3)).max()))
    return worst


def test_f16_weights_meet_the_bar():
    assert _worst_ratio(torch.float16) < 0.9


def test_bf16_weights_miss_the_bar():
    assert _worst_ratio(torch.bfloat16) > 1.0
