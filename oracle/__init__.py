"""CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference engine computes on its
attention path, so that the HIP kernels can be checked against it:

* ``oracle.attention``  -- float64 numpy restatement of every function on the
  path (decode, int8 dequant, paged gather, split-K merge, causal prefill,
  per-vector int8 quantisation).  This is the parity oracle.
* ``oracle.rope``       -- float32 numpy restatement of the fused q/k RoPE
  kernel (each product and sum rounded, output rounded to the input dtype).
* ``oracle.eager_path`` -- float32 torch restatement of the reference's own
  CPU/eager attention path (``repeat_interleave`` + SDPA), used as a second,
  library-backed cross-check and as the timed CPU baseline in ``bench.py``.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import anything under ``oracle/``, and only as the checker or the
reported CPU baseline.  The product path (the package next to this one) never
imports it and has no CPU fallback: it raises when its HIP library is missing.

How each oracle function is pinned (checks that do not retype its formula) is
listed in ``tests/test_oracle.py`` and ``tests/test_oracle_rope.py``; every function here has at least one such
check, so no function is "parity unpinned".
"""
