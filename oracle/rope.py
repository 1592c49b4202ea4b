"""CPU restatement of the reference's fused RoPE kernel (test oracle).

TEST INFRASTRUCTURE ONLY -- imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``; never by the product package.

Restates ``_rope_qk_fwd`` / ``_apply_qk`` (``kernels/rope_kernel.py:86-165``,
``193-258``): inputs converted to float32, ``out_a = x_a*cos - x_b*sin`` and
``out_b = x_b*cos + x_a*sin`` with each product and sum rounded to float32
(numpy never fuses), then rounded to the input dtype (nearest even).  Row
``r`` of the flattened ``B*T`` rows uses table row ``r % Tc``, and only the
first ``D/2`` table columns are read.  Pairs are ``(i, i + D/2)``
(split-half) or ``(2i, 2i + 1)`` (interleaved).

The reference compiles its kernel with Triton, which may contract
``x_a*cos - x_b*sin`` into a fused multiply-add; its results can then differ
from this restatement by one rounding of the fp32 intermediate (at most one
unit in the last place of the output dtype).  The HIP kernel follows this
restatement exactly, so the GPU tests compare bit for bit.

How ``rope_qk`` is pinned (checks that do not retype its formula) is in
``tests/test_oracle_rope.py``: transformers' Llama and GPT-J rotary functions
in float32 on the CPU (equal bit for bit), a float64/complex128 evaluation,
the identity at position 0, pairwise norm preservation, and the equality of
duplicated and half-width tables.
"""

from __future__ import annotations

import numpy as np

from .attention import round_to_dtype


def rope_qk(q, k, cos, sin, interleaved: bool = False, dtype: str = "float32"):
    """Rotate ``q (B, T, Hq, D)`` and ``k (B, T, Hkv, D)``; returns float32 arrays holding ``dtype`` values.

    ``q``/``k``/``cos``/``sin`` hold values already representable in their
    dtypes (float32 arrays); ``dtype`` is q/k's dtype, used for the output
    rounding.  ``cos``/``sin``: ``(Tc, D)`` or ``(Tc, D/2)``.
    """
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    cos = np.asarray(cos, dtype=np.float32)
    sin = np.asarray(sin, dtype=np.float32)
    B, T, _, D = q.shape
    half = D // 2
    rows = np.arange(B * T) % cos.shape[0]
    c = cos[rows, :half].reshape(B, T, 1, half)
    s = sin[rows, :half].reshape(B, T, 1, half)

    def one(x):
        if interleaved:
            xa, xb = x[..., 0::2], x[..., 1::2]
        else:
            xa, xb = x[..., :half], x[..., half:]
        oa = xa * c - xb * s
        ob = xb * c + xa * s
        out = np.empty_like(x)
        if interleaved:
            out[..., 0::2], out[..., 1::2] = oa, ob
        else:
            out[..., :half], out[..., half:] = oa, ob
        return round_to_dtype(out, dtype)

    return one(q), one(k)
