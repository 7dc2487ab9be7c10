"""The quantize kernels' division step (iq_quant.hip, div_rcp), checked on the CPU.

A group with a finite positive scale s divides its dividends (x - min for asym,
|x| for sym: finite fp16 values >= 0) through r = RN32(1/s) plus one fma
correction instead of a divide per value.  The claim the kernels rest on is
that its fp16 rounding equals the reference's fp16 division RN16(x / s)
(quant.py:69-71, 108-109) for every such pair; tests/quant_division.c checks
all 1,007,649,792 pairs of finite fp16 operands.  The GPU tests then compare
the kernels' codes bit for bit with the oracle and the golden vectors.
"""
import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is needed to build the checker")
def test_reciprocal_division_matches_fp16_division_exhaustively():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "quant_division")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", "-o", exe,
                        os.path.join(HERE, "quant_division.c"), "-lm"], check=True)
        r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip() == "pairs 1007649792 mismatches 0"
