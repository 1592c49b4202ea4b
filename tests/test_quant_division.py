"""CPU check of the int8 quantisation arithmetic the KV write kernel uses.

The kernel (``csrc/kv_write.hip``, ``div_by_scale``) evaluates ``x / scale``
as a reciprocal product plus one FMA correction instead of a full division.
``tests/quant_division_check.c`` compares the resulting int8 code with the
correctly rounded division of ``model/kv_cache.py:58-67`` over every bf16 and
fp16 ``|x| <= amax`` for a stride of amax patterns (stride 1 covers them all)
and over sampled fp32 pairs, including pairs within 3 ulps of a .5 tie.  The
GPU tests then check the kernel bit for bit against the oracle, which divides.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_reciprocal_fma_quotient_gives_division_codes(tmp_path):
    exe = tmp_path / "quant_division_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), os.path.join(HERE, "quant_division_check.c"),
                    "-lm"], check=True)
    r = subprocess.run([str(exe), "16", "4000000"], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "bf16:" in r.stdout and "fp16:" in r.stdout and "fp32:" in r.stdout
