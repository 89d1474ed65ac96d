"""Numerical identities the kernels rely on, checked exhaustively on the CPU.

* bf16 softmax (rowops.hip) forms y = r(e / s) -- XLA:CPU's bf16 divide: the
  IEEE f32 quotient rounded to bf16 -- without a division per element:
  q0 = RN(e * RN(1 / s)), corrected once (Markstein) with the exact FMA
  remainder.  numerics/bf16_quotient.c checks every positive bf16 e <= 1
  against every bf16 s in [1, 2^24] (a row's sum of exp(x - max) lies in
  [1, cols]); the bf16 results agree for all of them (the f32 values differ
  by one ulp for some tiny e, never across a bf16 rounding point).
"""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_bf16_softmax_quotient_matches_the_ieee_quotient(tmp_path):
    cc = shutil.which(os.environ.get("CC", "gcc"))
    if not cc:
        pytest.skip("no C compiler")
    exe = tmp_path / "bf16_quotient"
    subprocess.run([cc, "-O2", "-o", str(exe), os.path.join(HERE, "numerics", "bf16_quotient.c"), "-lm"],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
    assert r.stdout.startswith("0 of "), r.stdout
