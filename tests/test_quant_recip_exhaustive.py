"""The fp32-scale activation quant divides each value by its group scale
once per group (reciprocal) plus one FMA correction per value instead of an
IEEE division per value (e4m3_quant4_recip, device_common.hpp).  The fp32
quotient can then differ in its last bit, so this checks, over every input
the quantizer can see, that the e4m3 code never does: all positive finite
bf16 group maxima and all bf16 values inside each group (1.07e9 pairs, about
10 s on 8 threads).  A dropped correction or sign fix fails it."""
import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_reciprocal_quant_codes_equal_division_for_every_input():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "chk")
        subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
                        os.path.join(HERE, "quant_recip_check.c"), "-o", exe, "-lm"], check=True)
        r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    pairs, _, code_diff = (int(t) for t in r.stdout.split() if t.isdigit())
    assert pairs == 1065402240 and code_diff == 0, r.stdout
