"""Arithmetic identities the kernels rely on, checked on the CPU.

The binarizers divide row sums by the row's element count d (an integer in
1..1024: rows of up to 1024 columns) as x * (1/d) followed by one fma
correction (crb_amd/csrc/binarize.h, div_cnt).  That is the IEEE quotient
x / d bit for bit for every fp32 significand and every such d, which this
test checks exhaustively with gcc's fused multiply-add; scaling x by a power
of two scales each step exactly, so all normal x are covered."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_count_division_by_reciprocal_is_exact(tmp_path):
    exe = str(tmp_path / "div_exact")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-mfma", "-o", exe,
                    os.path.join(HERE, "div_exact.c"), "-lm"], check=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    assert out.strip() == "bad 0 of 8589934592", out
