"""The bf16 row quantizers replace x / s by Markstein's corrected quotient when the row
scale is at least 2^-120.  tests/quant_division_check.c walks every (bf16 amax, bf16 x)
pair with |x| <= amax and checks that the int8 code is the same either way."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).with_name("quant_division_check.c")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_quotient_gives_the_division_codes(tmp_path):
    exe = tmp_path / "qdc"
    base = ["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(SRC), "-lm"]
    if subprocess.run(base[:1] + ["-fopenmp"] + base[1:], capture_output=True).returncode:
        subprocess.run(base, check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    # the cut-off is needed: below it the two formulas do disagree
    assert "s >= 2^-120: 0;" in r.stdout and "below the cut-off: 0\n" not in r.stdout
