"""CPU check that the sibling kernel's reciprocal-plus-correction division
equals IEEE division for every bf16 scale (tests/native/scale_division_check.c)."""
import os
import shutil
import subprocess
import tempfile

import pytest

SRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "scale_division_check.c")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_division_matches_ieee():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "sdc")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-mfma", "-o", exe, SRC, "-lm"], check=True)
        res = subprocess.run([exe, "61"], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert " 0 mismatches" in res.stdout
