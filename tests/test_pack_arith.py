"""The fast packer's division-free arithmetic against IEEE float32, on the CPU.

``csrc/pack.hip`` computes the group scale with a Markstein step on the constant RN(1/qmax),
the codes with a Markstein-corrected reciprocal, and -- for groups whose scale is not clamped
above -- the code as the low byte of ``q + 2^23`` (round half to even by the add), Value words
by adding the shifted magic codes minus a constant.  ``pack_arith_check.c`` runs those steps in
the same order with C float32 and ``fmaf`` beside the reference's IEEE formula (layout.py:12-18)
over ranges of every magnitude, exact ties, repeated values and ranges around the 1e5 qmax
boundary.  The GPU tests check the kernel itself against the oracle and the golden data."""
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).with_name("pack_arith_check.c")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_and_magic_codes_match_ieee(tmp_path):
    exe = tmp_path / "pack_arith_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(SRC), "-lm"], check=True)
    out = subprocess.run([str(exe), "200000"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "differences 0" in out.stdout
    counts = out.stdout.split("magic ")[1]
    assert int(counts.split(",")[0]) > 0 and int(counts.split("clamped ")[1].split(")")[0]) > 0
